// Chunked (WY/UT) gated delta rule for prefill on gfx950 bf16 MFMA.
//
// For a chunk of C = 64 tokens starting from state S0 (Dv x Dk), with
// L_t = sum_{s<=t} log g_s, gamma_t = exp(L_t), e_t = exp(L_C - L_t):
//
//   A[t,i] = beta_t exp(L_t - L_i) (k_t . k_i)      (i < t)
//   U      = (I + A)^{-1} R,   R = diag(beta) (V - diag(gamma) K S0^T)
//   Y      = diag(gamma) Q S0^T + P U,   P[t,i] = exp(L_t - L_i) (q_t . k_i) (i <= t)
//   S_C    = gamma_C S0 + (diag(e) U)^T K
//
// Two launches:
//   chunk_prep  (grid: chunks x Hv)      -- all chunks in parallel: K K^T and
//               Q K^T on MFMA, the decay masks, and T = (I + A)^{-1} by a
//               blocked (16x16) forward substitution in fp32.  Writes T, P,
//               gamma, e, beta per (chunk, head) to the workspace.
//   chunk_scan  (grid: Dv/16 x Hv x seqs) -- sequential over the chunks of a
//               sequence; each workgroup owns 16 rows of the state, which
//               are independent in the recurrence, so the state chain of a
//               head is split over 8 workgroups.  Per chunk: X = [Q;K] S0^T,
//               R, U = T R, Y = gamma X_Q + P U, S update, all on MFMA.
//
// Precision: q, k, v are bf16 and enter MFMA exactly.  fp32 operands (S0, T,
// P, R, U) are split as hi + lo bf16 and multiplied in 2 (one exact operand)
// or 3 (both split; lo*lo dropped) passes, ~2^-16 relative per product, so
// the fp32 state meets a 1e-4 norm-wise tolerance.  Log-decay prefix sums
// are accumulated in fp64 so exp(L_t - L_i) does not lose digits when
// |L| is large.
#include "gdn_common.hpp"

namespace {

using namespace gdn;

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

constexpr int CH = 64;    // chunk length
constexpr int DK = 128;   // key head dim
constexpr int DV = 128;   // value head dim
constexpr int DVT = 16;   // state rows per scan workgroup
constexpr int KP = DK + 8;  // padded LDS row (bf16) for 128-wide rows
constexpr int CP = CH + 8;  // padded LDS row (bf16) for 64-wide rows

// Workspace record per (chunk, v-head).
constexpr size_t kOffT = 0;                        // float[64][64]  (I + A)^{-1}
constexpr size_t kOffP = kOffT + CH * CH * 4;      // float[64][64]  decayed Q K^T (lower)
constexpr size_t kOffGam = kOffP + CH * CH * 4;    // float[64]      exp(L_t)
constexpr size_t kOffE = kOffGam + CH * 4;         // float[64]      exp(L_C - L_t)
constexpr size_t kOffBeta = kOffE + CH * 4;        // float[64]
constexpr size_t kRecBytes = kOffBeta + CH * 4;    // 33536 (multiple of 256)

struct ChunkParams {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  const void* gx;
  const void* gy;
  const void* A_log;
  const void* dt_bias;
  int gate_mode, gate_dtype, param_dtype;
  const float* state_in;
  uint16_t* y;
  float* state_out;
  const int32_t* cu;  // [n_seqs + 1] or null
  int n_seqs;
  int T;              // tokens per sequence when cu == null
  int Hk, Hv, group;
  unsigned char* ws;
};

__device__ __forceinline__ f32x4 mfma16(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ uint16_t bf16_hi(float x) { return f32_to_bf16(x); }

__device__ __forceinline__ void split_bf16(float x, uint16_t& hi, uint16_t& lo) {
  hi = f32_to_bf16(x);
  lo = f32_to_bf16(x - bf16_to_f32(hi));
}

__device__ __forceinline__ bf16x8 lds8(const uint16_t* p) {
  return *reinterpret_cast<const bf16x8*>(p);
}

struct SeqRange {
  int64_t tok0;
  int len;
  int chunk0;  // global index of the sequence's first chunk
};

__device__ __forceinline__ int n_chunks(int len) { return (len + CH - 1) / CH; }

__device__ __forceinline__ SeqRange seq_range(const ChunkParams& p, int n) {
  SeqRange r;
  if (p.cu == nullptr) {
    r.tok0 = static_cast<int64_t>(n) * p.T;
    r.len = p.T;
    r.chunk0 = n * n_chunks(p.T);
    return r;
  }
  int base = 0;
  for (int m = 0; m < n; ++m) base += n_chunks(p.cu[m + 1] - p.cu[m]);
  r.tok0 = p.cu[n];
  r.len = p.cu[n + 1] - p.cu[n];
  r.chunk0 = base;
  return r;
}

// Global chunk index -> (first token, valid length).  False past the end.
__device__ __forceinline__ bool chunk_at(const ChunkParams& p, int c, int64_t& tok0, int& len) {
  if (p.cu == nullptr) {
    const int cps = n_chunks(p.T);
    if (cps == 0 || c >= p.n_seqs * cps) return false;
    const int n = c / cps, i = c % cps;
    tok0 = static_cast<int64_t>(n) * p.T + static_cast<int64_t>(i) * CH;
    len = min(CH, p.T - i * CH);
    return true;
  }
  int base = 0;
  for (int n = 0; n < p.n_seqs; ++n) {
    const int l = p.cu[n + 1] - p.cu[n];
    const int nc = n_chunks(l);
    if (c < base + nc) {
      const int i = c - base;
      tok0 = p.cu[n] + static_cast<int64_t>(i) * CH;
      len = min(CH, l - i * CH);
      return true;
    }
    base += nc;
  }
  return false;
}

// ------------------------------------------------------------ chunk_prep

__global__ __launch_bounds__(256) void chunk_prep_kernel(const ChunkParams p) {
  const int c = blockIdx.x;
  const int hv = blockIdx.y;
  int64_t tok0;
  int len;
  if (!chunk_at(p, c, tok0, len)) return;
  const int hk = hv / p.group;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;

  __shared__ __align__(16) uint16_t Ks[CH][KP];
  __shared__ __align__(16) uint16_t Qs[CH][KP];
  __shared__ float As[CH][CH + 1];
  __shared__ float Ti[CH][CH + 1];
  __shared__ float Ms[16][17];
  __shared__ double Ld[CH];
  __shared__ float Bs[CH];

  for (int i = tid; i < CH * (DK / 8); i += 256) {
    const int r = i / (DK / 8), cc = (i % (DK / 8)) * 8;
    uint4 kv = {0, 0, 0, 0}, qv = {0, 0, 0, 0};
    if (r < len) {
      const int64_t off = ((tok0 + r) * p.Hk + hk) * DK + cc;
      kv = *reinterpret_cast<const uint4*>(p.k + off);
      qv = *reinterpret_cast<const uint4*>(p.q + off);
    }
    *reinterpret_cast<uint4*>(&Ks[r][cc]) = kv;
    *reinterpret_cast<uint4*>(&Qs[r][cc]) = qv;
  }
  for (int i = tid; i < CH * (CH + 1); i += 256) (&Ti[0][0])[i] = 0.0f;

  unsigned char* rec = p.ws + (static_cast<size_t>(c) * p.Hv + hv) * kRecBytes;
  if (wave == 0) {
    float lg = 0.0f, bt = 0.0f;
    if (lane < len) {
      load_log_gates(p.gate_mode, p.gx, p.gy, p.gate_dtype, p.A_log, p.dt_bias, p.param_dtype,
                     (tok0 + lane) * p.Hv + hv, hv, lg, bt);
    }
    lg = fmaxf(lg, -1.0e30f);  // g = 0 (pre-transformed gates) stays finite
    double L = lg;
    for (int off = 1; off < 64; off <<= 1) {
      const double o = __shfl_up(L, off, 64);
      if (lane >= off) L += o;
    }
    Ld[lane] = L;
    Bs[lane] = bt;
    const double LC = __shfl(L, 63, 64);
    reinterpret_cast<float*>(rec + kOffGam)[lane] = expf(static_cast<float>(L));
    reinterpret_cast<float*>(rec + kOffE)[lane] = expf(static_cast<float>(LC - L));
    reinterpret_cast<float*>(rec + kOffBeta)[lane] = bt;
  }
  __syncthreads();

  // K K^T and Q K^T: wave w computes row block w (16 rows) x 4 column blocks.
  f32x4 kk[4], qk[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    kk[j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    qk[j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  }
  const int lr = lane & 15, lg8 = (lane >> 4) * 8;
#pragma unroll
  for (int s = 0; s < DK / 32; ++s) {
    const int kc = s * 32 + lg8;
    const bf16x8 ak = lds8(&Ks[16 * wave + lr][kc]);
    const bf16x8 aq = lds8(&Qs[16 * wave + lr][kc]);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const bf16x8 bk = lds8(&Ks[16 * j + lr][kc]);
      kk[j] = mfma16(ak, bk, kk[j]);
      qk[j] = mfma16(aq, bk, qk[j]);
    }
  }
  float* Pg = reinterpret_cast<float*>(rec + kOffP);
#pragma unroll
  for (int j = 0; j < 4; ++j) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int t = 16 * wave + 4 * (lane >> 4) + i;
      const int col = 16 * j + lr;
      const float dec = col <= t ? expf(static_cast<float>(Ld[t] - Ld[col])) : 0.0f;
      As[t][col] = col < t ? Bs[t] * dec * kk[j][i] : 0.0f;
      Pg[t * CH + col] = dec * qk[j][i];
    }
  }
  __syncthreads();

  // (I + A)^{-1}, A strictly lower.  Diagonal 16x16 blocks by forward
  // substitution (one lane per (block, column)).
  if (wave == 0) {
    const int base = 16 * (lane >> 4), j = lane & 15;
    float x[16];
#pragma unroll
    for (int t = 0; t < 16; ++t) {
      float acc = t == j ? 1.0f : 0.0f;
#pragma unroll
      for (int i = 0; i < t; ++i) acc = fmaf(-As[base + t][base + i], x[i], acc);
      x[t] = t < j ? 0.0f : acc;
    }
#pragma unroll
    for (int t = 0; t < 16; ++t) Ti[base + t][base + j] = x[t];
  }
  __syncthreads();
  // Off-diagonal blocks, by distance from the diagonal:
  //   T_IJ = -T_II * sum_{K=J}^{I-1} A_IK T_KJ
  {
    const int r = tid >> 4, cc = tid & 15;
    for (int lvl = 1; lvl < 4; ++lvl) {
      for (int I = lvl; I < 4; ++I) {
        const int J = I - lvl;
        float m = 0.0f;
        for (int Kb = J; Kb < I; ++Kb) {
#pragma unroll
          for (int x = 0; x < 16; ++x) m = fmaf(As[16 * I + r][16 * Kb + x], Ti[16 * Kb + x][16 * J + cc], m);
        }
        Ms[r][cc] = m;
        __syncthreads();
        float tv = 0.0f;
#pragma unroll
        for (int x = 0; x < 16; ++x) tv = fmaf(-Ti[16 * I + r][16 * I + x], Ms[x][cc], tv);
        Ti[16 * I + r][16 * J + cc] = tv;
        __syncthreads();
      }
    }
  }
  float* Tg = reinterpret_cast<float*>(rec + kOffT);
  for (int i = tid; i < CH * CH; i += 256) Tg[i] = Ti[i / CH][i % CH];
}

// ------------------------------------------------------------ chunk_scan

__global__ __launch_bounds__(256) void chunk_scan_kernel(const ChunkParams p) {
  const int dv0 = blockIdx.x * DVT;
  const int hv = blockIdx.y;
  const int seq = blockIdx.z;
  const int hk = hv / p.group;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int lr = lane & 15, lq = lane >> 4, lg8 = lq * 8;
  const SeqRange sr = seq_range(p, seq);
  const int nch = n_chunks(sr.len);

  __shared__ __align__(16) uint16_t Qs[CH][KP];
  __shared__ __align__(16) uint16_t Ks[CH][KP];
  __shared__ __align__(16) uint16_t KT[DK][CP];
  __shared__ __align__(16) uint16_t Th[CH][CP], Tl[CH][CP], Ph[CH][CP], Pl[CH][CP];
  __shared__ __align__(16) uint16_t Sh[DVT][KP], Sl[DVT][KP];
  __shared__ __align__(16) uint16_t Rh[DVT][CP], Rl[DVT][CP];
  __shared__ __align__(16) uint16_t Uh[DVT][CP], Ul[DVT][CP];
  __shared__ __align__(16) uint16_t Eh[DVT][CP], El[DVT][CP];
  __shared__ float Gs[CH], Es[CH], Bs[CH];

  // State tile (16 rows x 128): wave w holds columns [32w, 32w + 32) as two
  // 16x16 MFMA accumulator tiles; lane: rows 4*lq + i, column 16*j + lr.
  const int64_t srow0 = (static_cast<int64_t>(seq) * p.Hv + hv) * DV + dv0;
  f32x4 sacc[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int64_t idx = (srow0 + 4 * lq + i) * DK + 32 * wave + 16 * j + lr;
      sacc[j][i] = p.state_in != nullptr ? p.state_in[idx] : 0.0f;
    }
  }

  for (int ci = 0; ci < nch; ++ci) {
    const int64_t t0 = sr.tok0 + static_cast<int64_t>(ci) * CH;
    const int clen = min(CH, sr.len - ci * CH);
    const unsigned char* rec = p.ws + (static_cast<size_t>(sr.chunk0 + ci) * p.Hv + hv) * kRecBytes;

    __syncthreads();  // the previous chunk is done with every LDS buffer
    for (int i = tid; i < CH * (DK / 8); i += 256) {
      const int r = i / (DK / 8), cc = (i % (DK / 8)) * 8;
      uint4 kv = {0, 0, 0, 0}, qv = {0, 0, 0, 0};
      if (r < clen) {
        const int64_t off = ((t0 + r) * p.Hk + hk) * DK + cc;
        kv = *reinterpret_cast<const uint4*>(p.k + off);
        qv = *reinterpret_cast<const uint4*>(p.q + off);
      }
      *reinterpret_cast<uint4*>(&Ks[r][cc]) = kv;
      *reinterpret_cast<uint4*>(&Qs[r][cc]) = qv;
      const uint16_t* kh = reinterpret_cast<const uint16_t*>(&kv);
#pragma unroll
      for (int e = 0; e < 8; ++e) KT[cc + e][r] = kh[e];
    }
    {
      const float* Tg = reinterpret_cast<const float*>(rec + kOffT);
      const float* Pg = reinterpret_cast<const float*>(rec + kOffP);
      for (int i = tid; i < CH * CH / 4; i += 256) {
        const int r = (4 * i) / CH, cc = (4 * i) % CH;
        const f32x4 tv = *reinterpret_cast<const f32x4*>(Tg + 4 * i);
        const f32x4 pv = *reinterpret_cast<const f32x4*>(Pg + 4 * i);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          split_bf16(tv[e], Th[r][cc + e], Tl[r][cc + e]);
          split_bf16(pv[e], Ph[r][cc + e], Pl[r][cc + e]);
        }
      }
    }
    if (tid < CH) {
      Gs[tid] = reinterpret_cast<const float*>(rec + kOffGam)[tid];
      Es[tid] = reinterpret_cast<const float*>(rec + kOffE)[tid];
      Bs[tid] = reinterpret_cast<const float*>(rec + kOffBeta)[tid];
    }
#pragma unroll
    for (int j = 0; j < 2; ++j) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        split_bf16(sacc[j][i], Sh[4 * lq + i][32 * wave + 16 * j + lr],
                   Sl[4 * lq + i][32 * wave + 16 * j + lr]);
      }
    }
    __syncthreads();

    // X = [Q;K] S0^T for this wave's 16 tokens (rows) x 16 state rows (cols).
    f32x4 xq = {0.0f, 0.0f, 0.0f, 0.0f}, xk = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int s = 0; s < DK / 32; ++s) {
      const int kc = s * 32 + lg8;
      const bf16x8 aq = lds8(&Qs[16 * wave + lr][kc]);
      const bf16x8 ak = lds8(&Ks[16 * wave + lr][kc]);
      const bf16x8 bh = lds8(&Sh[lr][kc]);
      const bf16x8 bl = lds8(&Sl[lr][kc]);
      xq = mfma16(aq, bh, xq);
      xq = mfma16(aq, bl, xq);
      xk = mfma16(ak, bh, xk);
      xk = mfma16(ak, bl, xk);
    }
    // R = beta (V - gamma X_K), stored transposed: R^T[state row][token].
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int t = 16 * wave + 4 * lq + i;
      const float vv = t < clen ? bf16_to_f32(p.v[((t0 + t) * p.Hv + hv) * DV + dv0 + lr]) : 0.0f;
      const float r = Bs[t] * (vv - Gs[t] * xk[i]);
      split_bf16(r, Rh[lr][t], Rl[lr][t]);
    }
    __syncthreads();

    // U = T R: wave w -> tokens 16w..16w+15.
    f32x4 u = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int s = 0; s < CH / 32; ++s) {
      const int kc = s * 32 + lg8;
      const bf16x8 ah = lds8(&Th[16 * wave + lr][kc]);
      const bf16x8 al = lds8(&Tl[16 * wave + lr][kc]);
      const bf16x8 bh = lds8(&Rh[lr][kc]);
      const bf16x8 bl = lds8(&Rl[lr][kc]);
      u = mfma16(ah, bh, u);
      u = mfma16(ah, bl, u);
      u = mfma16(al, bh, u);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int t = 16 * wave + 4 * lq + i;
      split_bf16(u[i], Uh[lr][t], Ul[lr][t]);
      split_bf16(Es[t] * u[i], Eh[lr][t], El[lr][t]);
    }
    __syncthreads();

    // Y = gamma X_Q + P U for this wave's 16 tokens.
    f32x4 yacc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int s = 0; s < CH / 32; ++s) {
      const int kc = s * 32 + lg8;
      const bf16x8 ah = lds8(&Ph[16 * wave + lr][kc]);
      const bf16x8 al = lds8(&Pl[16 * wave + lr][kc]);
      const bf16x8 bh = lds8(&Uh[lr][kc]);
      const bf16x8 bl = lds8(&Ul[lr][kc]);
      yacc = mfma16(ah, bh, yacc);
      yacc = mfma16(ah, bl, yacc);
      yacc = mfma16(al, bh, yacc);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int t = 16 * wave + 4 * lq + i;
      if (t < clen) {
        const float yv = fmaf(Gs[t], xq[i], yacc[i]);
        p.y[((t0 + t) * p.Hv + hv) * DV + dv0 + lr] = f32_to_bf16(yv);
      }
    }

    // S = gamma_C S0 + (diag(e) U)^T K: wave w -> state columns [32w, 32w+32).
    const float gC = Gs[CH - 1];
#pragma unroll
    for (int j = 0; j < 2; ++j) sacc[j] *= gC;
#pragma unroll
    for (int s = 0; s < CH / 32; ++s) {
      const int kc = s * 32 + lg8;
      const bf16x8 eh = lds8(&Eh[lr][kc]);
      const bf16x8 el = lds8(&El[lr][kc]);
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const bf16x8 bk = lds8(&KT[32 * wave + 16 * j + lr][kc]);
        sacc[j] = mfma16(eh, bk, sacc[j]);
        sacc[j] = mfma16(el, bk, sacc[j]);
      }
    }
  }

#pragma unroll
  for (int j = 0; j < 2; ++j) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int64_t idx = (srow0 + 4 * lq + i) * DK + 32 * wave + 16 * j + lr;
      p.state_out[idx] = sacc[j][i];
    }
  }
}

int64_t max_chunks(int64_t n_seqs, int64_t n_tok, bool packed) {
  if (packed) return (n_tok + CH - 1) / CH + n_seqs;
  if (n_seqs == 0) return 0;
  const int64_t T = n_tok / n_seqs;
  return n_seqs * ((T + CH - 1) / CH);
}

}  // namespace

extern "C" size_t gdn_chunk_workspace_bytes(int64_t n_seqs, int64_t n_tok, int64_t Hv, int64_t Dk,
                                            int64_t Dv, int64_t chunk) {
  if (chunk != CH || Dk != DK || Dv != DV || n_seqs < 0 || n_tok < 0 || Hv <= 0) return 0;
  // Sized for packed sequences (an upper bound of the unpacked count too).
  const int64_t chunks = max_chunks(n_seqs, n_tok, true);
  return static_cast<size_t>(chunks) * static_cast<size_t>(Hv) * kRecBytes;
}

extern "C" int gdn_chunk_fwd(const void* q, const void* k, const void* v, int qkv_dtype,
                             int gate_mode, const void* gx, const void* gy, int gate_dtype,
                             const void* A_log, const void* dt_bias, int param_dtype,
                             const float* state_in, void* y, float* state_out,
                             const int32_t* cu_seqlens, int64_t n_seqs, int64_t n_tok, int64_t Hk,
                             int64_t Hv, int64_t Dk, int64_t Dv, int64_t chunk, void* workspace,
                             size_t workspace_bytes, void* stream) {
  using gdn_host::fail;
  if (chunk != CH) return fail(GDN_ERR_UNSUPPORTED, "gdn_chunk_fwd: chunk must be 64 (got %lld)", (long long)chunk);
  if (qkv_dtype != GDN_DTYPE_BF16) return fail(GDN_ERR_UNSUPPORTED, "gdn_chunk_fwd: q/k/v must be bf16");
  if (Dk != DK || Dv != DV)
    return fail(GDN_ERR_UNSUPPORTED, "gdn_chunk_fwd: built for Dk = Dv = 128 (got %lld, %lld)", (long long)Dk,
                (long long)Dv);
  if (n_seqs < 0 || n_tok < 0 || Hk <= 0 || Hv <= 0 || Hv % Hk != 0)
    return fail(GDN_ERR_INVALID, "gdn_chunk_fwd: bad sizes");
  if (gate_mode != GDN_GATES_RAW && gate_mode != GDN_GATES_PRE)
    return fail(GDN_ERR_INVALID, "gdn_chunk_fwd: bad gate_mode");
  if (!gdn_host::dtype_ok(gate_dtype) ||
      (gate_mode == GDN_GATES_RAW && (!gdn_host::dtype_ok(param_dtype) || !A_log || !dt_bias)))
    return fail(GDN_ERR_INVALID, "gdn_chunk_fwd: bad gate arguments");
  if (!q || !k || !v || !gx || !gy || !y || !state_out)
    return fail(GDN_ERR_INVALID, "gdn_chunk_fwd: q, k, v, gates, y and state_out are required");
  const bool packed = cu_seqlens != nullptr;
  if (!packed && n_seqs > 0 && n_tok % n_seqs != 0)
    return fail(GDN_ERR_INVALID, "gdn_chunk_fwd: n_tok=%lld is not n_seqs=%lld rows of equal length",
                (long long)n_tok, (long long)n_seqs);
  if (n_seqs == 0) return GDN_OK;
  const size_t need = gdn_chunk_workspace_bytes(n_seqs, n_tok, Hv, Dk, Dv, chunk);
  if (workspace == nullptr || workspace_bytes < need)
    return fail(GDN_ERR_INVALID, "gdn_chunk_fwd: workspace of %zu bytes is below the %zu needed", workspace_bytes,
                need);
  if (!gdn_host::aligned(workspace, 256) || !gdn_host::aligned(q, 16) || !gdn_host::aligned(k, 16) ||
      !gdn_host::aligned(state_in, 16) || !gdn_host::aligned(state_out, 16))
    return fail(GDN_ERR_INVALID, "gdn_chunk_fwd: misaligned pointer");
  if (n_tok > INT32_MAX / 2 || n_seqs > 65535 || Hv > 65535)
    return fail(GDN_ERR_UNSUPPORTED, "gdn_chunk_fwd: problem too large");

  ChunkParams p;
  p.q = static_cast<const uint16_t*>(q);
  p.k = static_cast<const uint16_t*>(k);
  p.v = static_cast<const uint16_t*>(v);
  p.gx = gx;
  p.gy = gy;
  p.A_log = A_log;
  p.dt_bias = dt_bias;
  p.gate_mode = gate_mode;
  p.gate_dtype = gate_dtype;
  p.param_dtype = param_dtype;
  p.state_in = state_in;
  p.y = static_cast<uint16_t*>(y);
  p.state_out = state_out;
  p.cu = cu_seqlens;
  p.n_seqs = static_cast<int>(n_seqs);
  p.T = packed ? 0 : static_cast<int>(n_tok / n_seqs);
  p.Hk = static_cast<int>(Hk);
  p.Hv = static_cast<int>(Hv);
  p.group = static_cast<int>(Hv / Hk);
  p.ws = static_cast<unsigned char*>(workspace);

  hipStream_t st = static_cast<hipStream_t>(stream);
  const int64_t chunks = max_chunks(n_seqs, n_tok, packed);
  if (chunks > 0) {
    hipLaunchKernelGGL(chunk_prep_kernel, dim3(static_cast<unsigned>(chunks), static_cast<unsigned>(Hv)),
                       dim3(256), 0, st, p);
    const int rc = gdn_host::check_launch("gdn_chunk_fwd/prep");
    if (rc != GDN_OK) return rc;
  }
  hipLaunchKernelGGL(chunk_scan_kernel,
                     dim3(static_cast<unsigned>(DV / DVT), static_cast<unsigned>(Hv), static_cast<unsigned>(n_seqs)),
                     dim3(256), 0, st, p);
  return gdn_host::check_launch("gdn_chunk_fwd/scan");
}
