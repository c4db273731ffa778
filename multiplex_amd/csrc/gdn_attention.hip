// Full-attention layers of the hybrid trunk and of the MTP draft head
// (Qwen3.5 gated attention) on gfx950.
//
//   attn_qk_kernel       one wave per (token, head): RMSNorm of q and k over
//                        the head dim (y = x / rms(x) * w), the rotary
//                        embedding of the first `rot` dims (rotate-half form,
//                        angle pos * base^(-2i/rot)), q to [B, T, Hq, D]; k and
//                        v appended to the KV cache [B, Hkv, cap, D] at
//                        positions pos0[b] .. pos0[b] + T - 1.
//   attn_fwd_kernel      causal GQA attention over the cache on bf16 MFMA
//                        with an online softmax in fp32.  The query rows of
//                        one kv-head are (token, q-head of its group) pairs,
//                        so the g = Hq / Hkv heads of a group share every K/V
//                        block a workgroup stages in LDS.  RT = 4: four waves
//                        own 16 rows each and walk the same 64-key blocks
//                        (prefill); RT = 1: one 16-row tile, each wave takes
//                        16 keys of every block (decode and draft verify,
//                        where a group has at most 16 rows), and the four
//                        partial softmax states merge in LDS at the end.
//                        Keys may also be split over workgroups; the partial
//                        states then go to a workspace and
//   attn_combine_kernel  merges them.
//   attn_prefill_kernel  long prefills (one key range, >= 512 rows per kv-head):
//                        128-row workgroups, 32 rows per wave, 64-key K / V
//                        blocks double-buffered in LDS (K by direct loads, V
//                        transposed on its way in), one barrier per block.
//                        The output is multiplied by sigmoid(gate) on the way
//                        out when a gate is given.
//   rms_norm_kernel      the layers' RMSNorm over the hidden size, optionally of
//                        a residual sum it also writes out.
//   silu_mul_kernel      the MLP's silu(gate) * up.
#include "gdn_common.hpp"

namespace {

using namespace gdn;

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef short i16x8 __attribute__((ext_vector_type(8)));
typedef __attribute__((address_space(3))) i16x4 lds_i16x4;
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr float kLog2e = 1.4426950408889634f;
constexpr int KB = 64;  // keys per staged block

__device__ __forceinline__ f32x4 mfma16(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ f32x4 mfma16k16(i16x4 a, i16x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ float sigmoid(float x) {
  return __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-x * kLog2e));
}

// ------------------------------------------------------------ attn_qk

struct QkParams {
  const uint16_t* qg;  // [B, T, Hq, 2D]: q, then the output gate, per head (token stride qg_ld)
  const uint16_t* kn;  // [B, T, Hkv, D] (token stride kv_ld)
  const uint16_t* vn;  // [B, T, Hkv, D] (token stride kv_ld)
  int64_t qg_ld, kv_ld;
  const void* qw;      // [D] q_norm weight
  const void* kw;      // [D] k_norm weight
  int wdt;
  const int32_t* pos0;  // [B] position of each row's first new token (its cache length)
  uint16_t* q;          // [B, T, Hq, D]
  uint16_t* kc;         // [B, Hkv, cap, D]
  uint16_t* vc;
  int B, T, Hq, Hkv, cap, rot;
  float eps, log2_base;
};

// A row's first position, clamped so that its T new tokens fit in the cache
// (offsets come from device memory and are not validated on the host).
__device__ __forceinline__ int first_pos(const int32_t* pos0, int b, int T, int cap) {
  return min(max(pos0[b], 0), cap - T);
}

template <int D>
__global__ __launch_bounds__(256) void attn_qk_kernel(const QkParams p) {
  constexpr int EPL = D / 64;  // elements per lane
  const int lane = threadIdx.x & 63;
  const int64_t item = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  const int heads = p.Hq + 2 * p.Hkv;  // q heads, k heads, v heads
  if (item >= static_cast<int64_t>(p.B) * p.T * heads) return;  // wave-uniform
  const int h = static_cast<int>(item % heads);
  const int64_t bt = item / heads;
  const int t = static_cast<int>(bt % p.T), b = static_cast<int>(bt / p.T);
  const int pos = first_pos(p.pos0, b, p.T, p.cap) + t;
  const int d0 = EPL * lane;

  const uint16_t* src;
  if (h < p.Hq) src = p.qg + bt * p.qg_ld + h * 2 * D;
  else if (h < p.Hq + p.Hkv) src = p.kn + bt * p.kv_ld + (h - p.Hq) * D;
  else src = p.vn + bt * p.kv_ld + (h - p.Hq - p.Hkv) * D;
  float x[EPL];
#pragma unroll
  for (int e = 0; e < EPL; ++e) x[e] = bf16_to_f32(src[d0 + e]);

  if (h >= p.Hq + p.Hkv) {  // v: into the cache as is
    uint16_t* dst = p.vc + ((static_cast<int64_t>(b) * p.Hkv + (h - p.Hq - p.Hkv)) * p.cap + pos) * D;
#pragma unroll
    for (int e = 0; e < EPL; ++e) dst[d0 + e] = src[d0 + e];
    return;
  }
  // RMSNorm, rounded to bf16 (the norm's output dtype)
  float ss = 0.0f;
#pragma unroll
  for (int e = 0; e < EPL; ++e) ss += x[e] * x[e];
  const float r = rsqrtf(wave_sum(ss) / D + p.eps);
  const void* w = h < p.Hq ? p.qw : p.kw;
#pragma unroll
  for (int e = 0; e < EPL; ++e) x[e] = bf16_to_f32(f32_to_bf16(x[e] * r * load_any(w, p.wdt, d0 + e)));
  // rotary embedding of dims [0, rot): d < half pairs with d + half
  const int half = p.rot / 2;
  const int shift = half / EPL;  // lanes between partners
  float y[EPL];
#pragma unroll
  for (int e = 0; e < EPL; ++e) {
    const bool lower = d0 < half;
    const float other = __shfl(x[e], lower ? lane + shift : lane - shift, 64);
    if (d0 < p.rot) {
      const int i = half > 0 ? (d0 + e) % half : 0;
      const float inv_freq = exp2f(-2.0f * static_cast<float>(i) / static_cast<float>(p.rot) * p.log2_base);
      float sn, cs;
      sincosf(static_cast<float>(pos) * inv_freq, &sn, &cs);
      y[e] = lower ? x[e] * cs - other * sn : x[e] * cs + other * sn;
    } else {
      y[e] = x[e];
    }
  }
  uint16_t* dst = h < p.Hq ? p.q + (bt * p.Hq + h) * D
                           : p.kc + ((static_cast<int64_t>(b) * p.Hkv + (h - p.Hq)) * p.cap + pos) * D;
#pragma unroll
  for (int e = 0; e < EPL; ++e) dst[d0 + e] = f32_to_bf16(y[e]);
}

// ------------------------------------------------------------ attn_fwd

struct AttnParams {
  const uint16_t* q;   // [B, T, Hq, D]
  const uint16_t* qg;  // gate source [B, T, Hq, 2D] (gate = second half of a head; token stride qg_ld) or null
  int64_t qg_ld;
  const uint16_t* kc;  // [B, Hkv, cap, D]
  const uint16_t* vc;
  const int32_t* pos0;  // [B]
  uint16_t* out;        // [B, T, Hq, D]
  float* part;          // split partials: O [B, Hkv, rows_pad, n_split, D], then m and l [.., n_split]
  int B, T, Hq, Hkv, cap;
  int n_split, split_len, rows_pad;
  float scale_log2;  // softmax scale * log2(e)
};

// Partial-state addressing for split keys.
__device__ __forceinline__ int64_t part_row(const AttnParams& p, int b, int hkv, int r) {
  return ((static_cast<int64_t>(b) * p.Hkv + hkv) * p.rows_pad + r) * p.n_split;
}

// Final value of one output element pair / quad: o / l, times the gate.
template <int D>
__device__ __forceinline__ void store_out4(const AttnParams& p, int b, int t, int hq, int d, f32x4 o, float inv_l) {
  const int64_t bt = static_cast<int64_t>(b) * p.T + t;
  const int64_t row = bt * p.Hq + hq;
  f32x4 y = o * inv_l;
  if (p.qg != nullptr) {
    const u32x2 gg = *reinterpret_cast<const u32x2*>(p.qg + bt * p.qg_ld + hq * 2 * D + D + d);
    y[0] *= sigmoid(__uint_as_float(gg.x << 16));
    y[1] *= sigmoid(__uint_as_float(gg.x & 0xffff0000u));
    y[2] *= sigmoid(__uint_as_float(gg.y << 16));
    y[3] *= sigmoid(__uint_as_float(gg.y & 0xffff0000u));
  }
  *reinterpret_cast<u32x2*>(p.out + row * D + d) = u32x2{pk_bf16(y[0], y[1]), pk_bf16(y[2], y[3])};
}

template <int D, int RT>
__global__ __launch_bounds__(256) void attn_fwd_kernel(const AttnParams p) {
  constexpr int KP = D + 8;   // K row stride (bf16): 16-byte fragment reads of 16 rows hit distinct banks
  constexpr int VP = D + 16;  // V row stride: the transposed reads of 4 rows hit distinct banks
  constexpr int KT = RT == 4 ? 4 : 1;  // 16-key tiles per wave and block
  constexpr int NS = D / 32;           // k-steps of q . k
  constexpr int NJ = D / 16;           // 16-wide d tiles of the output
  constexpr int CPT = KB * D / 8 / 256;  // 16-byte chunks per thread of a K (or V) block

  const int b = blockIdx.z;
  const int hkv = blockIdx.y % p.Hkv, rb = blockIdx.y / p.Hkv;
  const int split = blockIdx.x;
  const int g = p.Hq / p.Hkv;
  const int n_rows = p.T * g;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lr = lane & 15, lq = lane >> 4;
  const int p0 = first_pos(p.pos0, b, p.T, p.cap);

  const int row0 = rb * 16 * RT;
  const int t_last = min((row0 + 16 * RT - 1) / g, p.T - 1);
  const int k_lo = split * p.split_len;
  const int k_hi = min(p0 + t_last + 1, k_lo + p.split_len);  // keys of this workgroup: [k_lo, k_hi)
  const int rt = RT == 4 ? wave : 0;
  const int sub = RT == 4 ? 0 : wave;  // first 16-key tile of this wave in each block

  // this wave's 16 rows (lane lr's row): Q as the B operand of S^T = K Q^T
  const int r = row0 + 16 * rt + lr;
  const bool row_ok = r < n_rows;
  const int t = row_ok ? r / g : 0;
  const int hq = hkv * g + (row_ok ? r % g : 0);
  const int kmax = p0 + t;  // last key row r may see
  bf16x8 qf[NS];
  {
    const uint16_t* qrow = p.q + ((static_cast<int64_t>(b) * p.T + t) * p.Hq + hq) * D;
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      const u32x4 v = *reinterpret_cast<const u32x4*>(qrow + 32 * s + 8 * lq);
      qf[s] = __builtin_bit_cast(bf16x8, row_ok ? v : u32x4{0u, 0u, 0u, 0u});
    }
  }

  __shared__ __align__(16) unsigned char smem[KB * (KP + VP) * 2];
  uint16_t(*Ks)[KP] = reinterpret_cast<uint16_t(*)[KP]>(smem);
  uint16_t(*Vs)[VP] = reinterpret_cast<uint16_t(*)[VP]>(smem + KB * KP * 2);

  // the next block, in flight: chunk c = tid + 256 i is row c / (D/8), columns (c % (D/8)) * 8 ..
  // The cache is read with nontemporal loads: each step streams it once, and at
  // decode sizes (1 GB at B=64 and 4096 positions) it cannot stay in the
  // last-level cache, whose allocation on every read cost 15% (180.4 against
  // 152.8 us at B=64).
  u32x4 kr[CPT], vr[CPT];
  const int64_t head_base = (static_cast<int64_t>(b) * p.Hkv + hkv) * p.cap * D;
  auto load_blk = [&](int kb) {
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
      const int c = tid + 256 * i;
      const int row = c / (D / 8), col = (c % (D / 8)) * 8;
      const int key = kb + row;
      const int64_t off = head_base + static_cast<int64_t>(min(key, k_hi - 1)) * D + col;  // in bounds: k_hi <= cap
      kr[i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p.kc + off));
      vr[i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p.vc + off));
    }
  };
  auto store_blk = [&](int kb) {
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
      const int c = tid + 256 * i;
      const int row = c / (D / 8), col = (c % (D / 8)) * 8;
      const bool ok = kb + row < k_hi;  // keys past the range read as zero (the cache there is unset)
      const u32x4 z = {0u, 0u, 0u, 0u};
      *reinterpret_cast<u32x4*>(&Ks[row][col]) = ok ? kr[i] : z;
      *reinterpret_cast<u32x4*>(&Vs[row][col]) = ok ? vr[i] : z;
    }
  };

  float m = -INFINITY, l = 0.0f;  // running max (log2 units) and this lane's share of the sum
  f32x4 o[NJ];
#pragma unroll
  for (int j = 0; j < NJ; ++j) o[j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

  const int nblk = k_hi > k_lo ? (k_hi - k_lo + KB - 1) / KB : 0;
  if (nblk > 0) load_blk(k_lo);
  for (int blk = 0; blk < nblk; ++blk) {
    const int kb = k_lo + KB * blk;
    __syncthreads();  // the previous block's reads are done
    store_blk(kb);
    __syncthreads();
    if (blk + 1 < nblk) load_blk(kb + KB);

    // S^T = K Q^T for this wave's key tiles: lane (r, q) holds keys 16 kt + 4q + i of row r
    f32x4 sc[KT];
#pragma unroll
    for (int kt = 0; kt < KT; ++kt) {
      f32x4 a = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int s = 0; s < NS; ++s)
        a = mfma16(*reinterpret_cast<const bf16x8*>(&Ks[16 * (sub + kt) + lr][32 * s + 8 * lq]), qf[s], a);
      sc[kt] = a;
    }
    float mb = -INFINITY;
#pragma unroll
    for (int kt = 0; kt < KT; ++kt)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int key = kb + 16 * (sub + kt) + 4 * lq + i;
        const bool ok = row_ok && key <= kmax && key < k_hi;
        sc[kt][i] = ok ? sc[kt][i] * p.scale_log2 : -INFINITY;
        mb = fmaxf(mb, sc[kt][i]);
      }
    mb = fmaxf(mb, __shfl_xor(mb, 16, 64));
    mb = fmaxf(mb, __shfl_xor(mb, 32, 64));
    const float m_new = fmaxf(m, mb);
    const float m_use = m_new == -INFINITY ? 0.0f : m_new;
    const float alpha = __builtin_amdgcn_exp2f(m - m_use);
    m = m_new;
    float ps = 0.0f;
#pragma unroll
    for (int kt = 0; kt < KT; ++kt)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        sc[kt][i] = __builtin_amdgcn_exp2f(sc[kt][i] - m_use);
        ps += sc[kt][i];
      }
    l = l * alpha + ps;
#pragma unroll
    for (int j = 0; j < NJ; ++j) o[j] *= alpha;

    // O^T += V^T P^T (P as bf16; V^T by transposed LDS reads)
    if constexpr (RT == 4) {
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        // k-slots: keys 32 ks + 4q + (0..3), then 32 ks + 16 + 4q + (0..3) -- the rows of
        // accumulator tiles 2 ks and 2 ks + 1 held by lane group q
        const bf16x8 pb = __builtin_bit_cast(
            bf16x8, u32x4{pk_bf16(sc[2 * ks][0], sc[2 * ks][1]), pk_bf16(sc[2 * ks][2], sc[2 * ks][3]),
                          pk_bf16(sc[2 * ks + 1][0], sc[2 * ks + 1][1]), pk_bf16(sc[2 * ks + 1][2], sc[2 * ks + 1][3])});
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
          const uint16_t* va = &Vs[32 * ks + 4 * lq + (lr >> 2)][16 * j + 4 * (lr & 3)];
          const i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(va));
          const i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(va + 16 * VP));
          const bf16x8 vt = __builtin_bit_cast(bf16x8, i16x8(__builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7)));
          o[j] = mfma16(vt, pb, o[j]);
        }
      }
    } else {
      const u32x2 pw = {pk_bf16(sc[0][0], sc[0][1]), pk_bf16(sc[0][2], sc[0][3])};
      const i16x4 pb = __builtin_bit_cast(i16x4, pw);
#pragma unroll
      for (int j = 0; j < NJ; ++j) {
        const uint16_t* va = &Vs[16 * sub + 4 * lq + (lr >> 2)][16 * j + 4 * (lr & 3)];
        o[j] = mfma16k16(__builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(va)), pb, o[j]);
      }
    }
  }
  l += __shfl_xor(l, 16, 64);
  l += __shfl_xor(l, 32, 64);

  const bool split_out = p.n_split > 1;
  if constexpr (RT == 4) {
    // lane (r, q) holds O[row r][16 j + 4 q + i]
    if (!row_ok) return;
    if (split_out) {
      const int64_t pr = part_row(p, b, hkv, r) + split;
      float* po = p.part + pr * D;
#pragma unroll
      for (int j = 0; j < NJ; ++j) *reinterpret_cast<f32x4*>(po + 16 * j + 4 * lq) = o[j];
      if (lq == 0) {
        float* ml = p.part + static_cast<int64_t>(p.B) * p.Hkv * p.rows_pad * p.n_split * D;
        const int64_t n_part = static_cast<int64_t>(p.B) * p.Hkv * p.rows_pad * p.n_split;
        ml[pr] = m;
        ml[n_part + pr] = l;
      }
      return;
    }
    const float inv_l = l > 0.0f ? 1.0f / l : 0.0f;
#pragma unroll
    for (int j = 0; j < NJ; ++j) store_out4<D>(p, b, t, hq, 16 * j + 4 * lq, o[j], inv_l);
  } else {
    // merge the four waves' states for the tile's 16 rows (the K/V buffers are free)
    __syncthreads();
    float* Os = reinterpret_cast<float*>(smem);  // [4][16][D]
    float* Ms = Os + 4 * 16 * D;                 // [4][16]
    float* Ls = Ms + 4 * 16;
    static_assert((4 * 16 * D + 2 * 64) * 4 <= KB * (KP + VP) * 2, "merge buffers must fit in the K/V blocks");
#pragma unroll
    for (int j = 0; j < NJ; ++j) *reinterpret_cast<f32x4*>(&Os[(wave * 16 + lr) * D + 16 * j + 4 * lq]) = o[j];
    if (lq == 0) {
      Ms[wave * 16 + lr] = m;
      Ls[wave * 16 + lr] = l;
    }
    __syncthreads();
    // thread: row tid / 16, columns (tid % 16) * D/16 ..
    constexpr int CW = D / 16;
    const int mr = tid >> 4, c0 = (tid & 15) * CW;
    const int rr = row0 + mr;
    if (rr >= n_rows) return;
    float mw[4], ms = -INFINITY;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      mw[w] = Ms[w * 16 + mr];
      ms = fmaxf(ms, mw[w]);
    }
    const float m_use = ms == -INFINITY ? 0.0f : ms;
    float sw[4], lsum = 0.0f;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      sw[w] = __builtin_amdgcn_exp2f(mw[w] - m_use);
      lsum += sw[w] * Ls[w * 16 + mr];
    }
    if (split_out) {
      const int64_t pr = part_row(p, b, hkv, rr) + split;
      float* po = p.part + pr * D;
#pragma unroll
      for (int c = 0; c < CW; c += 4) {
        f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int w = 0; w < 4; ++w) acc += sw[w] * *reinterpret_cast<const f32x4*>(&Os[(w * 16 + mr) * D + c0 + c]);
        *reinterpret_cast<f32x4*>(po + c0 + c) = acc;
      }
      if ((tid & 15) == 0) {
        float* ml = p.part + static_cast<int64_t>(p.B) * p.Hkv * p.rows_pad * p.n_split * D;
        const int64_t n_part = static_cast<int64_t>(p.B) * p.Hkv * p.rows_pad * p.n_split;
        ml[pr] = ms;
        ml[n_part + pr] = lsum;
      }
      return;
    }
    const float inv_l = lsum > 0.0f ? 1.0f / lsum : 0.0f;
    const int tt = rr / g, hh = hkv * g + rr % g;
#pragma unroll
    for (int c = 0; c < CW; c += 4) {
      f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int w = 0; w < 4; ++w) acc += sw[w] * *reinterpret_cast<const f32x4*>(&Os[(w * 16 + mr) * D + c0 + c]);
      store_out4<D>(p, b, tt, hh, c0 + c, acc, inv_l);
    }
  }
}

// Long causal prefills (one key range, at least kPrefillRows rows per kv-head):
// a workgroup owns 128 rows, four waves of 32, so every K or V fragment a
// wave reads from LDS feeds two 16-row MFMA tiles.  64-key blocks are double-
// buffered in LDS and a block costs one barrier:
//   K  goes in by direct global -> LDS loads (each lane's 16 bytes land at
//      16 * lane past the wave's base), rows of D bf16 whose 16-byte granules
//      are XOR-swizzled by (key & 7), so the fragment reads of 8 consecutive
//      keys hit distinct banks;
//   V  is transposed in registers on its way in: Vt[d][position], with the
//      keys of each 32-key group in the k-slot order of the P^T operand
//      (position 8q + 4h + i holds key 16h + 4q + i), so that a V^T fragment
//      is one 16-byte read, like K's; rows of 64 positions whose 16-byte
//      granules are XOR-swizzled by (d & 7), which keeps both the fragment
//      reads and the 8-byte transposed writes free of bank conflicts.  (Transposed LDS reads of a [key][d]
//      block deliver about 45 bytes per clock per CU, against 128 for 16-byte
//      reads.)
// The softmax max is raised only when a row's block max exceeds it by more
// than 8 (log2 units; P stays below 2^8), which skips the rescale of the
// output on most blocks, and only blocks that cross the diagonal or the end
// of the keys are masked.  Workgroups with the longest key ranges go first.
// 16 bytes per lane from global memory straight into LDS at lds_base + 16 * lane (lds_base wave-
// uniform).  Issued from inline assembly: the compiler's wait insertion, seeing an LDS DMA in a
// loop, would otherwise drain every LDS read with lgkmcnt(0).  It increments vmcnt like any load;
// the caller waits for it (vmcnt(0)) before the barrier that publishes the block.
__device__ __forceinline__ void lds_dma16(const void* gptr, uint32_t lds_base) {
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off"
               :
               : "v"(gptr), "s"(lds_base)
               : "memory", "m0");
}

// Max / sum over the four 16-lane rows of a wave (lanes r, r + 16, r + 32, r + 48), by the
// gfx950 row-swap moves (VALU, no LDS round trip): permlane16_swap(x, x) yields the even and the
// odd rows, permlane32_swap(x, x) the low and the high halves, each in both places.
__device__ __forceinline__ float rows_max(float x) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}
__device__ __forceinline__ float rows_sum(float x) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

constexpr int kPrefillRows = 512;  // rows (tokens x heads of a group) per kv-head from which it is used
constexpr int PR = 128;            // rows per workgroup
constexpr int VTP = KB;            // Vt row stride (bf16); 16-byte granules XOR-swizzled by (d & 7)

template <int D>
__global__ __launch_bounds__(256) void attn_prefill_kernel(const AttnParams p) {
  constexpr int NS = D / 32;                  // k-steps of q . k
  constexpr int NJ = D / 16;                  // 16-wide d tiles of the output
  constexpr int KG = D / 8;                   // 16-byte granules per K row
  constexpr int KDMA = KB * KG / 256;         // direct loads per thread and K block
  constexpr int VPAIRS = (KB / 4) * KG / 256;  // (key quad, d octet) pairs per thread and V block
  constexpr int KSTAGE = KB * D * 2;          // bytes
  constexpr int VSTAGE = D * VTP * 2;
  static_assert(KDMA * 256 == KB * KG && VPAIRS * 256 == (KB / 4) * KG, "block must split evenly over 256 threads");

  __shared__ __align__(16) unsigned char smem[2 * (KSTAGE + VSTAGE)];

  const int b = blockIdx.z;
  const int n_rb = gridDim.x / p.Hkv;
  const int hkv = blockIdx.x % p.Hkv;
  const int rb = n_rb - 1 - static_cast<int>(blockIdx.x) / p.Hkv;  // longest key ranges first
  const int g = p.Hq / p.Hkv;
  const int n_rows = p.T * g;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lr = lane & 15, lq = lane >> 4;
  const int p0 = first_pos(p.pos0, b, p.T, p.cap);

  const int row0 = rb * PR;
  const int t_last = min((row0 + PR - 1) / g, p.T - 1);
  const int k_hi = min(p0 + t_last + 1, p.split_len);  // keys of this workgroup: [0, k_hi)
  const int k_free = min(p0 + row0 / g + 1, k_hi);      // keys below this are visible to every row

  // the wave's two 16-row tiles; rows past the end compute on q = 0 and are not stored
  int t[2], hq[2], kmax[2];
  bool row_ok[2];
  bf16x8 qf[2][NS];
#pragma unroll
  for (int rt = 0; rt < 2; ++rt) {
    const int r = row0 + 32 * wave + 16 * rt + lr;
    row_ok[rt] = r < n_rows;
    t[rt] = row_ok[rt] ? r / g : p.T - 1;
    hq[rt] = hkv * g + (row_ok[rt] ? r % g : 0);
    kmax[rt] = p0 + t[rt];
    const uint16_t* qrow = p.q + ((static_cast<int64_t>(b) * p.T + t[rt]) * p.Hq + hq[rt]) * D;
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      const u32x4 v = *reinterpret_cast<const u32x4*>(qrow + 32 * s + 8 * lq);
      qf[rt][s] = __builtin_bit_cast(bf16x8, row_ok[rt] ? v : u32x4{0u, 0u, 0u, 0u});
    }
  }

  const uint16_t* kc_head = p.kc + (static_cast<int64_t>(b) * p.Hkv + hkv) * p.cap * D;
  const uint16_t* vc_head = p.vc + (static_cast<int64_t>(b) * p.Hkv + hkv) * p.cap * D;
  // K block kb -> stage st: thread tid's load i fills physical granule i * 256 + tid, which is row
  // i * KR + tid / KG, granule (tid % KG) ^ (row & 7) of the block (the swizzle does not depend on i)
  constexpr int KR = 256 / KG;
  const int k_row0 = tid / KG;
  const int k_off = k_row0 * D + (((tid % KG) ^ (k_row0 & 7)) * 8);
  // LDS address of the wave's 1 KB slice of load 0 in stage 0
  const uint32_t k_lds = __builtin_amdgcn_readfirstlane(
      static_cast<uint32_t>(reinterpret_cast<uintptr_t>(smem)) + wave * 1024);
  // keys past the range re-read the last one (in bounds; they are masked)
  auto k_dma = [&](int kb, int st, int i) {
    const int key = min(kb + i * KR + k_row0, k_hi - 1);
    lds_dma16(kc_head + static_cast<int64_t>(key) * D + (k_off - k_row0 * D), k_lds + st * KSTAGE + i * 4096);
  };
  // V block kb -> registers: pair i is key quad tid % 16 (4 rows) x d octet i * 16 + tid / 16
  const int v_kq = tid % (KB / 4), v_dq = tid / (KB / 4);
  u32x4 vr[VPAIRS][4];
  auto v_load = [&](int kb, int i, int e) {
    const int key = min(kb + 4 * v_kq + e, k_hi - 1);
    vr[i][e] = *reinterpret_cast<const u32x4*>(vc_head + static_cast<int64_t>(key) * D + (v_dq + i * 16) * 8);
  };
  // registers -> Vt stage st: for each of the octet's 8 d, the quad's 4 keys as one 8-byte write
  const int v_pos = 32 * (v_kq >> 3) + 8 * (v_kq & 3) + 4 * ((v_kq >> 2) & 1);
  const int v_gran = v_pos >> 3, v_half = v_pos & 7;  // the position's granule and offset in it
  auto v_store = [&](int st, int i, int m) {  // d rows 8 (v_dq + 16 i) + 2m, + 2m + 1 (d & 7 = 2m, 2m + 1)
    uint16_t* Vt = reinterpret_cast<uint16_t*>(smem + 2 * KSTAGE + st * VSTAGE) + (8 * (v_dq + i * 16)) * VTP + v_half;
    const uint32_t k0 = vr[i][0][m], k1 = vr[i][1][m], k2 = vr[i][2][m], k3 = vr[i][3][m];
    const u32x2 even = {(k0 & 0xffffu) | (k1 << 16), (k2 & 0xffffu) | (k3 << 16)};
    const u32x2 odd = {(k0 >> 16) | (k1 & 0xffff0000u), (k2 >> 16) | (k3 & 0xffff0000u)};
    *reinterpret_cast<u32x2*>(Vt + (2 * m) * VTP + ((v_gran ^ (2 * m)) << 3)) = even;
    *reinterpret_cast<u32x2*>(Vt + (2 * m + 1) * VTP + ((v_gran ^ (2 * m + 1)) << 3)) = odd;
  };

  float m[2] = {-INFINITY, -INFINITY}, l[2] = {0.0f, 0.0f};
  f32x4 o[2][NJ];
#pragma unroll
  for (int rt = 0; rt < 2; ++rt)
#pragma unroll
    for (int j = 0; j < NJ; ++j) o[rt][j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

  // K fragment (tile kt, k-step s) of lane (r, q): row 16 kt + r, granule (4s + q) ^ (r & 7)
  // = 8 (s >> 1) + 4 ((s & 1) ^ x2) + (q ^ x01) with x = r & 7: one base for even s, one for odd,
  // each plus 64 (s & ~1) bytes
  const int x2 = (lr >> 2) & 1, y01 = lq ^ (lr & 3);
  const int kfe = lr * (D * 2) + (4 * x2 + y01) * 16, kfo = lr * (D * 2) + (4 * (x2 ^ 1) + y01) * 16;
  // V^T fragment (j, ks) of lane (r, q): d row 16 j + r, positions 32 ks + 8q .., granule (4 ks + q) ^ (r & 7)
  const int vfo0 = lr * (VTP * 2) + (4 * x2 + y01) * 16, vfo1 = lr * (VTP * 2) + (4 * (x2 ^ 1) + y01) * 16;

  const int nblk = (k_hi + KB - 1) / KB;  // >= 1: k_hi > p0 + row0 / g >= 0
#pragma unroll
  for (int i = 0; i < KDMA; ++i) k_dma(0, 0, i);
#pragma unroll
  for (int i = 0; i < VPAIRS; ++i) {
#pragma unroll
    for (int e = 0; e < 4; ++e) v_load(0, i, e);
#pragma unroll
    for (int m = 0; m < 4; ++m) v_store(0, i, m);
  }
  for (int blk = 0; blk < nblk; ++blk) {
    const int kb = KB * blk, st = blk & 1;
    __builtin_amdgcn_s_waitcnt(0);  // this thread's direct loads of block blk have landed
    __syncthreads();                // everyone's have, Vt[st] is written, stage st ^ 1 is free
    // the next block's K and V go in while this one computes: one K load and one V load per k-step of
    // S^T, V stored (transposed) during O^T; the last block re-reads itself into the free stage (never
    // read) so that no load sits behind a branch
    const int kb_next = blk + 1 < nblk ? kb + KB : kb;

    // S^T = K Q^T: lane (r, q) holds keys 16 kt + 4q + i of row r, for both row tiles
    const unsigned char* Ks = smem + st * KSTAGE;
    auto k_frag = [&](int s, int kt) {
      return *reinterpret_cast<const bf16x8*>(Ks + ((s & 1) ? kfo : kfe) + kt * 16 * (D * 2) + (s & ~1) * 64);
    };
    f32x4 sc[2][4];
#pragma unroll
    for (int kt = 0; kt < 4; ++kt) sc[0][kt] = sc[1][kt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    bf16x8 kf[2][4];  // the fragments of k-step s, and those of s + 1 in flight
#pragma unroll
    for (int kt = 0; kt < 4; ++kt) kf[0][kt] = k_frag(0, kt);
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      if (s + 1 < NS) {
#pragma unroll
        for (int kt = 0; kt < 4; ++kt) kf[(s + 1) & 1][kt] = k_frag(s + 1, kt);
      }
      static_assert(KDMA == NS, "one K load per k-step");
      k_dma(kb_next, st ^ 1, s);
      if (s < 4 * VPAIRS) v_load(kb_next, s / 4, s % 4);
#pragma unroll
      for (int kt = 0; kt < 4; ++kt) {
        sc[0][kt] = mfma16(kf[s & 1][kt], qf[0][s], sc[0][kt]);
        sc[1][kt] = mfma16(kf[s & 1][kt], qf[1][s], sc[1][kt]);
      }
    }
    // issue order: k-step s + 1's four fragment reads ahead of k-step s's eight products
    __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      if (s + 1 < NS) __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
      if (s < 4 * VPAIRS) __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x008, 8, 0);
    }

    if (kb + KB > k_free) {
#pragma unroll
      for (int rt = 0; rt < 2; ++rt)
#pragma unroll
        for (int kt = 0; kt < 4; ++kt)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int key = kb + 16 * kt + 4 * lq + i;
            if (!(key <= kmax[rt] && key < k_hi)) sc[rt][kt][i] = -INFINITY;
          }
    }
    float mb[2];
    bool grow = false;
#pragma unroll
    for (int rt = 0; rt < 2; ++rt) {
      float x = -INFINITY;
#pragma unroll
      for (int kt = 0; kt < 4; ++kt)
#pragma unroll
        for (int i = 0; i < 4; ++i) x = fmaxf(x, sc[rt][kt][i]);
      mb[rt] = rows_max(x) * p.scale_log2;
      grow |= mb[rt] > m[rt] + 8.0f;
    }
    if (__builtin_amdgcn_ballot_w64(grow) != 0) {
#pragma unroll
      for (int rt = 0; rt < 2; ++rt) {
        const float m_new = fmaxf(m[rt], mb[rt]);
        const float alpha = __builtin_amdgcn_exp2f(m[rt] - m_new);
        m[rt] = m_new;
        l[rt] *= alpha;
#pragma unroll
        for (int j = 0; j < NJ; ++j) o[rt][j] *= alpha;
      }
    }
    // P = exp2(s * scale - m) as the B operand of O^T += V^T P^T: k-slots 8q .. 8q+3 are keys
    // 32 ks + 4q + (0..3) (accumulator tile 2 ks), 8q+4 .. 8q+7 are keys 32 ks + 16 + 4q + (0..3)
    bf16x8 pb[2][2];
#pragma unroll
    for (int rt = 0; rt < 2; ++rt) {
      float ps = 0.0f;
#pragma unroll
      for (int kt = 0; kt < 4; ++kt)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          sc[rt][kt][i] = __builtin_amdgcn_exp2f(fmaf(sc[rt][kt][i], p.scale_log2, -m[rt]));
          ps += sc[rt][kt][i];
        }
      l[rt] += ps;
#pragma unroll
      for (int ks = 0; ks < 2; ++ks)
        pb[rt][ks] = __builtin_bit_cast(
            bf16x8, u32x4{pk_bf16(sc[rt][2 * ks][0], sc[rt][2 * ks][1]), pk_bf16(sc[rt][2 * ks][2], sc[rt][2 * ks][3]),
                          pk_bf16(sc[rt][2 * ks + 1][0], sc[rt][2 * ks + 1][1]),
                          pk_bf16(sc[rt][2 * ks + 1][2], sc[rt][2 * ks + 1][3])});
    }

    // O^T += V^T P^T
    const unsigned char* Vt = smem + 2 * KSTAGE + st * VSTAGE;
    constexpr int NF = 2 * NJ;  // V^T fragments per block: (ks, j) = (f / NJ, f % NJ)
    constexpr int VPF = 4;      // fragments in flight
    auto v_frag = [&](int f) {
      return *reinterpret_cast<const bf16x8*>(Vt + (f / NJ ? vfo1 : vfo0) + (f % NJ) * 16 * (VTP * 2));
    };
    bf16x8 vf[VPF];
#pragma unroll
    for (int f = 0; f < VPF; ++f) vf[f] = v_frag(f);
#pragma unroll
    for (int f = 0; f < NF; ++f) {
      const bf16x8 a = vf[f % VPF];
      if (f + VPF < NF) vf[f % VPF] = v_frag(f + VPF);
      const int j = f % NJ, ks = f / NJ;
      o[0][j] = mfma16(a, pb[0][ks], o[0][j]);
      o[1][j] = mfma16(a, pb[1][ks], o[1][j]);
      // the next block's V into the free stage
      if (f % 2 == 1 && f / 2 < 4 * VPAIRS) v_store(st ^ 1, f / 8, (f / 2) % 4);
    }
    // issue order: fragment f + VPF read ahead of fragment f's two products
    __builtin_amdgcn_sched_group_barrier(0x100, VPF, 1);
#pragma unroll
    for (int f = 0; f < NF; ++f) {
      if (f + VPF < NF) __builtin_amdgcn_sched_group_barrier(0x100, 1, 1);
      __builtin_amdgcn_sched_group_barrier(0x008, 2, 1);
    }

  }

#pragma unroll
  for (int rt = 0; rt < 2; ++rt) {
    const float lt = rows_sum(l[rt]);
    if (!row_ok[rt]) continue;
    const float inv_l = lt > 0.0f ? 1.0f / lt : 0.0f;
#pragma unroll
    for (int j = 0; j < NJ; ++j) store_out4<D>(p, b, t[rt], hq[rt], 16 * j + 4 * lq, o[rt][j], inv_l);
  }
}

// One wave per (row, kv-head, batch row): the split partials of a row merged.
template <int D>
__global__ __launch_bounds__(256) void attn_combine_kernel(const AttnParams p) {
  const int lane = threadIdx.x & 63;
  const int g = p.Hq / p.Hkv;
  const int n_rows = p.T * g;
  const int64_t item = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (item >= static_cast<int64_t>(p.B) * p.Hkv * n_rows) return;
  const int r = static_cast<int>(item % n_rows);
  const int hkv = static_cast<int>((item / n_rows) % p.Hkv);
  const int b = static_cast<int>(item / (static_cast<int64_t>(n_rows) * p.Hkv));
  const int64_t n_part = static_cast<int64_t>(p.B) * p.Hkv * p.rows_pad * p.n_split;
  const float* ml = p.part + n_part * D;
  const int64_t pr = part_row(p, b, hkv, r);
  float ms = -INFINITY;
  for (int s = 0; s < p.n_split; ++s) ms = fmaxf(ms, ml[pr + s]);
  const float m_use = ms == -INFINITY ? 0.0f : ms;
  constexpr int EPL = D / 64;
  f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
  float lsum = 0.0f;
  for (int s = 0; s < p.n_split; ++s) {
    const float w = __builtin_amdgcn_exp2f(ml[pr + s] - m_use);
    lsum += w * ml[n_part + pr + s];
    const float* po = p.part + (pr + s) * D + EPL * lane;
    if constexpr (EPL == 4) {
      acc += w * *reinterpret_cast<const f32x4*>(po);
    } else {
      acc[0] += w * po[0];
      acc[1] += w * po[1];
    }
  }
  const float inv_l = lsum > 0.0f ? 1.0f / lsum : 0.0f;
  const int t = r / g, hq = hkv * g + r % g;
  if constexpr (EPL == 4) {
    store_out4<D>(p, b, t, hq, EPL * lane, acc, inv_l);
  } else {
    const int64_t bt = static_cast<int64_t>(b) * p.T + t;
    const int64_t row = bt * p.Hq + hq;
    float y0 = acc[0] * inv_l, y1 = acc[1] * inv_l;
    const int d = EPL * lane;
    if (p.qg != nullptr) {
      const uint16_t* gp = p.qg + bt * p.qg_ld + hq * 2 * D + D + d;
      y0 *= sigmoid(bf16_to_f32(gp[0]));
      y1 *= sigmoid(bf16_to_f32(gp[1]));
    }
    *reinterpret_cast<uint32_t*>(p.out + row * D + d) = pk_bf16(y0, y1);
  }
}

// ------------------------------------------------------------ rms_norm

// Eight weights from index i (a multiple of 8) as floats: one 16-byte load for
// bf16 / fp16, two for fp32 (the branch is uniform).
__device__ __forceinline__ void load_w8(const void* w, int wdt, int i, float out[8]) {
  if (wdt == GDN_DTYPE_F32) {
    const f32x4 a = *reinterpret_cast<const f32x4*>(static_cast<const float*>(w) + i);
    const f32x4 b = *reinterpret_cast<const f32x4*>(static_cast<const float*>(w) + i + 4);
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      out[k] = a[k];
      out[4 + k] = b[k];
    }
  } else {
    const u32x4 v = *reinterpret_cast<const u32x4*>(static_cast<const uint16_t*>(w) + i);
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const uint16_t lo = static_cast<uint16_t>(v[k] & 0xffffu), hi = static_cast<uint16_t>(v[k] >> 16);
      out[2 * k] = wdt == GDN_DTYPE_BF16 ? bf16_to_f32(lo) : f16_to_f32(lo);
      out[2 * k + 1] = wdt == GDN_DTYPE_BF16 ? bf16_to_f32(hi) : f16_to_f32(hi);
    }
  }
}

// One workgroup per row; 8 bf16 elements per thread and chunk, chunk c of
// thread t at 8 t + 2048 c.  With a residual, the row is h = bf16(x + res)
// (written to h_out when given) and y = norm(h); y's rows are y_ld elements
// apart.  The first kRegChunks chunks of h stay in registers between the sum
// of squares and the output (one pass over memory up to D = 8192); chunks
// beyond are read again, from h_out when this thread wrote them (h_out may
// alias x), else recomputed.
constexpr int kRegChunks = 4;
__global__ __launch_bounds__(256) void rms_norm_kernel(const uint16_t* x, const uint16_t* res, uint16_t* h_out,
                                                       const void* w, int wdt, uint16_t* y, int64_t y_ld, int D,
                                                       float eps) {
  const int64_t row = blockIdx.x;
  const uint16_t* xr = x + row * D;
  const uint16_t* rr = res != nullptr ? res + row * D : nullptr;
  auto load_h = [&](int c) {
    u32x4 v = *reinterpret_cast<const u32x4*>(xr + c);
    if (rr != nullptr) {
      const u32x4 r = *reinterpret_cast<const u32x4*>(rr + c);
#pragma unroll
      for (int k = 0; k < 4; ++k)
        v[k] = pk_bf16(__uint_as_float(v[k] << 16) + __uint_as_float(r[k] << 16),
                       __uint_as_float(v[k] & 0xffff0000u) + __uint_as_float(r[k] & 0xffff0000u));
    }
    return v;
  };
  auto sq = [](u32x4 v) {
    float ss = 0.0f;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const float a = __uint_as_float(v[k] << 16), bb = __uint_as_float(v[k] & 0xffff0000u);
      ss += a * a + bb * bb;
    }
    return ss;
  };
  const int c0 = 8 * threadIdx.x;
  u32x4 hv[kRegChunks];
  float wv[kRegChunks][8];
  float ss = 0.0f;
#pragma unroll
  for (int j = 0; j < kRegChunks; ++j) {
    const int c = c0 + 2048 * j;
    if (c < D) {
      hv[j] = load_h(c);
      load_w8(w, wdt, c, wv[j]);
    }
  }
#pragma unroll
  for (int j = 0; j < kRegChunks; ++j) {
    const int c = c0 + 2048 * j;
    if (c < D) {
      if (h_out != nullptr) *reinterpret_cast<u32x4*>(h_out + row * D + c) = hv[j];
      ss += sq(hv[j]);
    }
  }
  for (int c = c0 + 2048 * kRegChunks; c < D; c += 2048) {
    const u32x4 v = load_h(c);
    if (h_out != nullptr) *reinterpret_cast<u32x4*>(h_out + row * D + c) = v;
    ss += sq(v);
  }
  __shared__ float part[4];
  ss = wave_sum(ss);
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = ss;
  __syncthreads();
  const float r = rsqrtf((part[0] + part[1] + part[2] + part[3]) / D + eps);
  auto out8 = [&](int c, u32x4 v, const float* wk) {
    u32x4 o;
#pragma unroll
    for (int k = 0; k < 4; ++k)
      o[k] = pk_bf16(__uint_as_float(v[k] << 16) * r * wk[2 * k], __uint_as_float(v[k] & 0xffff0000u) * r * wk[2 * k + 1]);
    *reinterpret_cast<u32x4*>(y + row * y_ld + c) = o;
  };
#pragma unroll
  for (int j = 0; j < kRegChunks; ++j) {
    const int c = c0 + 2048 * j;
    if (c < D) out8(c, hv[j], wv[j]);
  }
  for (int c = c0 + 2048 * kRegChunks; c < D; c += 2048) {
    const u32x4 v = h_out != nullptr ? *reinterpret_cast<const u32x4*>(h_out + row * D + c) : load_h(c);
    float wk[8];
    load_w8(w, wdt, c, wk);
    out8(c, v, wk);
  }
}

// ------------------------------------------------------------ silu_mul

// out[r, i] = silu(gu[r, i]) * gu[r, I + i]; 8 elements per thread.
__global__ __launch_bounds__(256) void silu_mul_kernel(const uint16_t* gu, uint16_t* out, int64_t rows, int I) {
  const int64_t i8 = (static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x) * 8;
  if (i8 >= rows * I) return;
  const int64_t r = i8 / I;
  const int c = static_cast<int>(i8 % I);
  const u32x4 gv = *reinterpret_cast<const u32x4*>(gu + r * 2 * I + c);
  const u32x4 uv = *reinterpret_cast<const u32x4*>(gu + r * 2 * I + I + c);
  u32x4 o;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const float g0 = __uint_as_float(gv[k] << 16), g1 = __uint_as_float(gv[k] & 0xffff0000u);
    const float u0 = __uint_as_float(uv[k] << 16), u1 = __uint_as_float(uv[k] & 0xffff0000u);
    o[k] = pk_bf16(silu(g0) * u0, silu(g1) * u1);
  }
  *reinterpret_cast<u32x4*>(out + i8) = o;
}

int64_t attn_rows_pad(int64_t T, int64_t Hq, int64_t Hkv, int rt) {
  const int64_t n_rows = T * (Hq / Hkv);
  const int64_t tile = 16 * rt;
  return (n_rows + tile - 1) / tile * tile;
}

int attn_rt(int64_t T, int64_t Hq, int64_t Hkv) { return T * (Hq / Hkv) <= 16 ? 1 : 4; }

}  // namespace

extern "C" size_t gdn_attn_workspace_bytes(int64_t B, int64_t T, int64_t Hq, int64_t Hkv, int64_t D,
                                           int64_t n_split) {
  if (B <= 0 || T <= 0 || Hq <= 0 || Hkv <= 0 || Hq % Hkv != 0 || D <= 0 || n_split < 1) return 0;
  if (n_split == 1) return 0;
  const int64_t rows_pad = attn_rows_pad(T, Hq, Hkv, attn_rt(T, Hq, Hkv));
  return static_cast<size_t>(B * Hkv * rows_pad * n_split) * (D + 2) * sizeof(float);
}

extern "C" int gdn_attn_qk(const void* qg, int64_t qg_ld, const void* k_new, const void* v_new, int64_t kv_ld,
                           const void* q_norm_w, const void* k_norm_w, int w_dtype, float eps, const int32_t* pos0,
                           void* q_out, void* k_cache, void* v_cache, int64_t B, int64_t T, int64_t Hq, int64_t Hkv,
                           int64_t D, int64_t cap, int64_t rot, float rope_base, void* stream) {
  using gdn_host::fail;
  if (D != 128 && D != 256) return fail(GDN_ERR_UNSUPPORTED, "gdn_attn_qk: head dim must be 128 or 256 (got %lld)", (long long)D);
  if (B < 0 || T < 0 || Hq <= 0 || Hkv <= 0 || Hq % Hkv != 0 || cap < T || cap > INT32_MAX)
    return fail(GDN_ERR_INVALID, "gdn_attn_qk: bad sizes");
  if (rot < 0 || rot > D || rot % (2 * (D / 64)) != 0 || (rot > 0 && (rot / 2) % (D / 64) != 0))
    return fail(GDN_ERR_UNSUPPORTED, "gdn_attn_qk: rotary dims %lld not supported for head dim %lld", (long long)rot,
                (long long)D);
  if (!gdn_host::dtype_ok(w_dtype) || !(rope_base > 0.0f) || !(eps >= 0.0f))
    return fail(GDN_ERR_INVALID, "gdn_attn_qk: bad norm weight dtype, eps or rope base");
  if (B * T == 0) return GDN_OK;
  if (!qg || !k_new || !v_new || !q_norm_w || !k_norm_w || !pos0 || !q_out || !k_cache || !v_cache)
    return fail(GDN_ERR_INVALID, "gdn_attn_qk: null pointer");
  if (B * T * (Hq + 2 * Hkv) > INT32_MAX) return fail(GDN_ERR_UNSUPPORTED, "gdn_attn_qk: problem too large");
  if (qg_ld == 0) qg_ld = 2 * Hq * D;
  if (kv_ld == 0) kv_ld = Hkv * D;
  if (qg_ld < 2 * Hq * D || kv_ld < Hkv * D) return fail(GDN_ERR_INVALID, "gdn_attn_qk: token strides below the rows");
  QkParams p;
  p.qg = static_cast<const uint16_t*>(qg);
  p.kn = static_cast<const uint16_t*>(k_new);
  p.vn = static_cast<const uint16_t*>(v_new);
  p.qg_ld = qg_ld;
  p.kv_ld = kv_ld;
  p.qw = q_norm_w;
  p.kw = k_norm_w;
  p.wdt = w_dtype;
  p.pos0 = pos0;
  p.q = static_cast<uint16_t*>(q_out);
  p.kc = static_cast<uint16_t*>(k_cache);
  p.vc = static_cast<uint16_t*>(v_cache);
  p.B = static_cast<int>(B);
  p.T = static_cast<int>(T);
  p.Hq = static_cast<int>(Hq);
  p.Hkv = static_cast<int>(Hkv);
  p.cap = static_cast<int>(cap);
  p.rot = static_cast<int>(rot);
  p.eps = eps;
  p.log2_base = log2f(rope_base);
  const int64_t waves = B * T * (Hq + 2 * Hkv);
  const dim3 grid(static_cast<unsigned>((waves + 3) / 4));
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (D == 256) hipLaunchKernelGGL(attn_qk_kernel<256>, grid, dim3(256), 0, st, p);
  else hipLaunchKernelGGL(attn_qk_kernel<128>, grid, dim3(256), 0, st, p);
  return gdn_host::check_launch("gdn_attn_qk");
}

extern "C" int gdn_attn_fwd(const void* q, const void* qg, int64_t qg_ld, const void* k_cache, const void* v_cache,
                            const int32_t* pos0, void* out, float scale, int64_t B, int64_t T, int64_t Hq,
                            int64_t Hkv, int64_t D, int64_t cap, int64_t kv_len_max, int64_t n_split,
                            void* workspace, size_t workspace_bytes, void* stream) {
  using gdn_host::fail;
  if (D != 128 && D != 256) return fail(GDN_ERR_UNSUPPORTED, "gdn_attn_fwd: head dim must be 128 or 256 (got %lld)", (long long)D);
  if (B < 0 || T < 0 || Hq <= 0 || Hkv <= 0 || Hq % Hkv != 0 || cap < T || cap > INT32_MAX || n_split < 1 ||
      n_split > 65535 || kv_len_max < T || kv_len_max > cap)
    return fail(GDN_ERR_INVALID, "gdn_attn_fwd: bad sizes (kv_len_max must lie in [T, cap])");
  if (!(scale > 0.0f)) return fail(GDN_ERR_INVALID, "gdn_attn_fwd: scale must be positive");
  if (B * T == 0) return GDN_OK;
  if (!q || !k_cache || !v_cache || !pos0 || !out) return fail(GDN_ERR_INVALID, "gdn_attn_fwd: null pointer");
  if (qg_ld == 0) qg_ld = 2 * Hq * D;
  if (qg && qg_ld < 2 * Hq * D) return fail(GDN_ERR_INVALID, "gdn_attn_fwd: gate token stride below the row");
  if (!gdn_host::aligned(q, 16) || !gdn_host::aligned(k_cache, 16) || !gdn_host::aligned(v_cache, 16) ||
      !gdn_host::aligned(out, 8) || (qg && (!gdn_host::aligned(qg, 8) || qg_ld % 4 != 0)))
    return fail(GDN_ERR_INVALID, "gdn_attn_fwd: misaligned pointer");
  const int rt = attn_rt(T, Hq, Hkv);
  const int64_t rows_pad = attn_rows_pad(T, Hq, Hkv, rt);
  const int64_t n_rb = rows_pad / (16 * rt);
  if (B > 65535 || Hkv * n_rb > INT32_MAX || B * Hkv * rows_pad * n_split * (D + 2) > (int64_t(1) << 40))
    return fail(GDN_ERR_UNSUPPORTED, "gdn_attn_fwd: problem too large");
  const size_t need = gdn_attn_workspace_bytes(B, T, Hq, Hkv, D, n_split);
  if (need > 0 && (workspace == nullptr || workspace_bytes < need || !gdn_host::aligned(workspace, 16)))
    return fail(GDN_ERR_INVALID, "gdn_attn_fwd: workspace of %zu bytes is below the %zu needed for %lld splits",
                workspace_bytes, need, (long long)n_split);
  AttnParams p;
  p.q = static_cast<const uint16_t*>(q);
  p.qg = static_cast<const uint16_t*>(qg);
  p.qg_ld = qg_ld;
  p.kc = static_cast<const uint16_t*>(k_cache);
  p.vc = static_cast<const uint16_t*>(v_cache);
  p.pos0 = pos0;
  p.out = static_cast<uint16_t*>(out);
  p.part = static_cast<float*>(workspace);
  p.B = static_cast<int>(B);
  p.T = static_cast<int>(T);
  p.Hq = static_cast<int>(Hq);
  p.Hkv = static_cast<int>(Hkv);
  p.cap = static_cast<int>(cap);
  p.n_split = static_cast<int>(n_split);
  p.split_len = static_cast<int>(((kv_len_max + n_split - 1) / n_split + KB - 1) / KB * KB);
  p.rows_pad = static_cast<int>(rows_pad);
  p.scale_log2 = scale * kLog2e;
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (n_split == 1 && T * (Hq / Hkv) >= kPrefillRows) {
    const int64_t n_prb = (T * (Hq / Hkv) + PR - 1) / PR;
    if (Hkv * n_prb > INT32_MAX) return fail(GDN_ERR_UNSUPPORTED, "gdn_attn_fwd: problem too large");
    const dim3 pgrid(static_cast<unsigned>(Hkv * n_prb), 1, static_cast<unsigned>(B));
    if (D == 256) hipLaunchKernelGGL(attn_prefill_kernel<256>, pgrid, dim3(256), 0, st, p);
    else hipLaunchKernelGGL(attn_prefill_kernel<128>, pgrid, dim3(256), 0, st, p);
    return gdn_host::check_launch("gdn_attn_fwd/prefill");
  }
  const dim3 grid(static_cast<unsigned>(n_split), static_cast<unsigned>(Hkv * n_rb), static_cast<unsigned>(B));
  if (D == 256) {
    if (rt == 4) hipLaunchKernelGGL((attn_fwd_kernel<256, 4>), grid, dim3(256), 0, st, p);
    else hipLaunchKernelGGL((attn_fwd_kernel<256, 1>), grid, dim3(256), 0, st, p);
  } else {
    if (rt == 4) hipLaunchKernelGGL((attn_fwd_kernel<128, 4>), grid, dim3(256), 0, st, p);
    else hipLaunchKernelGGL((attn_fwd_kernel<128, 1>), grid, dim3(256), 0, st, p);
  }
  int rc = gdn_host::check_launch("gdn_attn_fwd");
  if (rc != GDN_OK || n_split == 1) return rc;
  const int64_t waves = B * Hkv * T * (Hq / Hkv);
  const dim3 cgrid(static_cast<unsigned>((waves + 3) / 4));
  if (D == 256) hipLaunchKernelGGL(attn_combine_kernel<256>, cgrid, dim3(256), 0, st, p);
  else hipLaunchKernelGGL(attn_combine_kernel<128>, cgrid, dim3(256), 0, st, p);
  return gdn_host::check_launch("gdn_attn_fwd/combine");
}

extern "C" int gdn_rms_norm(const void* x, const void* res, void* h_out, const void* w, int w_dtype, void* y,
                            int64_t y_ld, int64_t rows, int64_t D, float eps, void* stream) {
  using gdn_host::fail;
  if (rows < 0 || D <= 0 || D % 8 != 0 || D > INT32_MAX || rows > INT32_MAX)
    return fail(GDN_ERR_INVALID, "gdn_rms_norm: bad sizes (D must be a multiple of 8)");
  if (y_ld == 0) y_ld = D;
  if (y_ld < D || y_ld % 8 != 0) return fail(GDN_ERR_INVALID, "gdn_rms_norm: y row stride must be >= D and a multiple of 8");
  if (!gdn_host::dtype_ok(w_dtype) || !(eps >= 0.0f)) return fail(GDN_ERR_INVALID, "gdn_rms_norm: bad weight dtype or eps");
  if (rows == 0) return GDN_OK;
  if (!x || !w || !y) return fail(GDN_ERR_INVALID, "gdn_rms_norm: null pointer");
  if (!gdn_host::aligned(x, 16) || !gdn_host::aligned(y, 16) || !gdn_host::aligned(w, 16) ||
      (res && !gdn_host::aligned(res, 16)) || (h_out && !gdn_host::aligned(h_out, 16)))
    return fail(GDN_ERR_INVALID, "gdn_rms_norm: misaligned pointer");
  hipLaunchKernelGGL(rms_norm_kernel, dim3(static_cast<unsigned>(rows)), dim3(256), 0, static_cast<hipStream_t>(stream),
                     static_cast<const uint16_t*>(x), static_cast<const uint16_t*>(res), static_cast<uint16_t*>(h_out),
                     w, w_dtype, static_cast<uint16_t*>(y), y_ld, static_cast<int>(D), eps);
  return gdn_host::check_launch("gdn_rms_norm");
}

extern "C" int gdn_silu_mul(const void* gate_up, void* out, int64_t rows, int64_t I, void* stream) {
  using gdn_host::fail;
  if (rows < 0 || I <= 0 || I % 8 != 0 || I > INT32_MAX) return fail(GDN_ERR_INVALID, "gdn_silu_mul: bad sizes (I must be a multiple of 8)");
  if (rows == 0) return GDN_OK;
  if (!gate_up || !out) return fail(GDN_ERR_INVALID, "gdn_silu_mul: null pointer");
  if (!gdn_host::aligned(gate_up, 16) || !gdn_host::aligned(out, 16)) return fail(GDN_ERR_INVALID, "gdn_silu_mul: misaligned pointer");
  const int64_t n8 = rows * I / 8;
  if ((n8 + 255) / 256 > INT32_MAX) return fail(GDN_ERR_UNSUPPORTED, "gdn_silu_mul: problem too large");
  hipLaunchKernelGGL(silu_mul_kernel, dim3(static_cast<unsigned>((n8 + 255) / 256)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), static_cast<const uint16_t*>(gate_up), static_cast<uint16_t*>(out),
                     rows, static_cast<int>(I));
  return gdn_host::check_launch("gdn_silu_mul");
}
