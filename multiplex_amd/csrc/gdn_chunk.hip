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
//   chunk_prep  (grid: chunks x Hv)      -- every chunk in parallel: K K^T
//               and Q K^T on MFMA, the decay masks, T = (I + A)^{-1} by a
//               blocked (16x16) forward substitution in fp32.  Writes T and
//               P as hi/lo bf16 planes (MFMA-ready) plus gamma, e, beta.
//   chunk_scan  (8 workgroups per head)  -- sequential over the chunks of a
//               sequence; a workgroup owns 16 rows of the state (rows are
//               independent in the recurrence, so one head's chain is split
//               over 8 workgroups).  Per chunk: X = [Q;K] S0^T, R, U = T R,
//               Y = gamma X_Q + P U, S update, all on MFMA, with one
//               cross-wave exchange (the state) per chunk.  The operands of
//               chunk c+1 are loaded into registers while chunk c computes.
//
// Precision: q, k, v are bf16 and enter MFMA exactly.  fp32 operands (S0, T,
// P, R, U) are split as hi + lo bf16 and multiplied in 2 (one exact operand)
// or 3 (both split; lo*lo dropped) passes, ~2^-16 relative per product, so
// the fp32 state meets a 1e-4 norm-wise tolerance.  Log-decay prefix sums
// are accumulated in fp64 so exp(L_t - L_i) keeps its digits when |L| is
// large.
#include <mutex>

#include "gdn_common.hpp"

namespace {

using namespace gdn;

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

constexpr int CH = 64;      // chunk length
constexpr int DK = 128;     // key head dim
constexpr int DV = 128;     // value head dim
constexpr int DVT = 16;     // state rows per scan workgroup
constexpr int KP = DK + 8;  // padded LDS row (bf16) for 128-wide rows
constexpr int CP = CH + 8;  // padded LDS row (bf16) for 64-wide rows
constexpr double kLog2e = 1.4426950408889634;

// Workspace record per (chunk, v-head).  Matrices are stored as MFMA
// fragments: the 16 x 32 block (row block rb, column block cb) of a matrix
// with n column blocks is 1 KB at ((rb * n + cb) * 64 + lane) * 16 bytes, lane
// (r % 16) + 16 * ((c % 32) / 8) holding columns c .. c+7 of row r -- exactly
// the A/B operand registers of a 16x16x32 MFMA, so a wave loads a fragment
// with one contiguous 1 KB read.
constexpr size_t kOffTh = 0;                        // bf16 64x64   hi((I + A)^{-1})
constexpr size_t kOffTl = kOffTh + CH * CH * 2;     // bf16 64x64   lo
constexpr size_t kOffPh = kOffTl + CH * CH * 2;     // bf16 64x64   hi(decayed Q K^T)
constexpr size_t kOffPl = kOffPh + CH * CH * 2;     // bf16 64x64   lo
// K^T, K and Q are per k-head: written into the record of its first v-head.
constexpr size_t kOffKT = kOffPl + CH * CH * 2;     // bf16 128x64  K^T
constexpr size_t kOffKf = kOffKT + DK * CH * 2;     // bf16 64x128  K
constexpr size_t kOffQf = kOffKf + CH * DK * 2;     // bf16 64x128  Q
constexpr size_t kOffGam = kOffQf + CH * DK * 2;    // float[64]    exp(L_t)
constexpr size_t kOffE = kOffGam + CH * 4;          // float[64]    exp(L_C - L_t)
constexpr size_t kOffBeta = kOffE + CH * 4;         // float[64]
constexpr size_t kRecBytes = kOffBeta + CH * 4;     // 82688 (multiple of 256)
// float[64] exp(L_t) for y, 0 at a masked token: in fragment 1 of the P hi
// plane (rows 0-15, columns 32-63: above the diagonal, so never written as
// P nor read by the scan), which keeps the record at 323 x 256 bytes (a
// stride of 81 KiB measurably slowed the fused prep).
constexpr size_t kOffGy = kOffPh + 1024;

// Element offset of (r, c) in the fragment layout of a matrix with ncb
// 32-column blocks.
__host__ __device__ constexpr int frag_elem(int r, int c, int ncb) {
  return (((r >> 4) * ncb + (c >> 5)) * 64 + (r & 15) + 16 * ((c & 31) >> 3)) * 8 + (c & 7);
}
static_assert(kRecBytes % 256 == 0, "workspace records must stay 256-byte aligned");

struct ChunkParams {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  GateArgs ga;
  const float* state_in;
  uint16_t* y;
  float* state_out;
  const int32_t* state_index;  // slot of each sequence in pooled states, or null
  int n_slots;
  const int32_t* cu;  // [n_seqs + 1] or null
  int n_seqs;
  int n_tok;          // tokens in all sequences
  int T;              // tokens per sequence when cu == null
  int Hk, Hv, group;
  unsigned char* ws;
  int32_t* order;     // [n_seqs] packed sequences longest first (in the workspace), or null
  const uint8_t* mask;  // [n_tok] token mask (0 = masked: the state is kept, y = 0), or null
  // The conv prologue fused into the prep (chunk_prep_kernel with CONV): q,
  // k and v are formed from the mixed qkv rows; the prep writes v to v_out
  // (p.v points at it, for the scan) and the sequences' new conv states.
  const uint16_t* qkv;
  int64_t qkv_ld;         // elements from one qkv row to the next
  const void* conv_w;     // [C][4] taps, bf16 or fp32
  const uint16_t* cs_in;  // [n_seqs][3][C], or null (zeros)
  uint16_t* cs_out;       // [n_seqs][3][C], or null
  uint16_t* v_out;        // [n_tok][Hv][DV]
  int C;                  // qkv channels: 2 Hk DK + Hv DV
  float conv_eps;
};

typedef __attribute__((address_space(1))) const uint8_t gbl_u8;

// Packed calls of 2..kOrderMax sequences order them by length, so the scan
// deals the longest chains out first; above that, sequence order.
constexpr int kOrderMax = 1024;

__device__ __forceinline__ f32x4 mfma16(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ void split_bf16(float x, uint16_t& hi, uint16_t& lo) {
  hi = f32_to_bf16(x);
  lo = f32_to_bf16(x - bf16_to_f32(hi));
}

__device__ __forceinline__ bf16x8 lds8(const uint16_t* p) {
  return *reinterpret_cast<const bf16x8*>(p);
}

typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef short i16x8 __attribute__((ext_vector_type(8)));
typedef __attribute__((address_space(3))) i16x4 lds_i16x4;

// K^T as an MFMA A-fragment from K rows in LDS ([token][dk], row stride KP),
// by two transposed reads (ds_read_b64_tr_b16).  Within each 16-lane group,
// lane i of a transposed read receives element i % 4 of the 4 read by lane
// 4e + i / 4, for e = 0..3.  Lane (r, q) here passes &K[t0 + r / 4][d0 + 4 (r % 4)]
// (t0 = the fragment's first token + 8 q, d0 = its first dk), so it receives
// K[t0 + e][d0 + r]: tokens t0 .. t0+3 of dk d0 + r, then t0+4 .. t0+7 from
// the rows 4 further on -- the 8 k-slots of row d0 + r of the fragment.
__device__ __forceinline__ bf16x8 kt_frag(const uint16_t* p) {
  const i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(p));
  const i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(p + 4 * KP));
  return __builtin_bit_cast(bf16x8, i16x8(__builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7)));
}


typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// hi = bf16(x), lo = bf16(x - hi) for 4 values, as two 8-byte LDS stores.
// The residual takes hi back from the packed pair (shift / mask) rather than
// converting each value a second time.
__device__ __forceinline__ void split4_store(f32x4 x, uint16_t* hi, uint16_t* lo) {
  const uint32_t h01 = pk_bf16(x[0], x[1]), h23 = pk_bf16(x[2], x[3]);
  const float r0 = x[0] - __builtin_bit_cast(float, h01 << 16);
  const float r1 = x[1] - __builtin_bit_cast(float, h01 & 0xffff0000u);
  const float r2 = x[2] - __builtin_bit_cast(float, h23 << 16);
  const float r3 = x[3] - __builtin_bit_cast(float, h23 & 0xffff0000u);
  *reinterpret_cast<u32x2*>(hi) = u32x2{h01, h23};
  *reinterpret_cast<u32x2*>(lo) = u32x2{pk_bf16(r0, r1), pk_bf16(r2, r3)};
}

struct SeqRange {
  int64_t tok0;
  int len;
  int chunk0;  // global index of the sequence's first chunk
};

__device__ __forceinline__ int n_chunks(int len) { return (len + CH - 1) / CH; }

// Workgroups are dispatched to the 8 XCDs round-robin by linear block id.
// This maps block id (below n, the number of work blocks) -> work index so
// that each XCD gets one contiguous range of work indices (whose consumers
// of the same data then share that XCD's L2).  Identity when n does not
// split evenly.
__device__ __forceinline__ int xcd_work_index(int n) {
  constexpr int kXcds = 8;
  const int b = blockIdx.x;
  if (n % kXcds != 0) return b;
  return (b % kXcds) * (n / kXcds) + b / kXcds;
}

// Chunk slots of packed sequences.  Sequence n owns the slots from
// cu[n] / CH + n on: with cu[n] = aC + r and a length of bC + s,
// a + ceil((bC + s) / C) <= floor(((a + b)C + r + s) / C) + 1, so the slots
// of consecutive sequences never overlap, and the last one is below
// n_tok / CH + n_seqs (the workspace bound).  A sequence's first slot is
// then one load away, with no sum over the sequences before it; the slots
// a sequence leaves unused hold no record.
//
// Offsets from a device tensor are not validated on the host, so every read
// of the table clamps: sequence n spans [start(n), end(n)) with
// start(n) = clamp(cu[n], 0, n_tok) and end(n) = clamp(cu[n+1], start(n), n_tok).
// A bad table then gives wrong rows, but every token, record and slot index
// stays within the bounds above.
__device__ __forceinline__ int cu_start(const ChunkParams& p, int n) { return min(max(p.cu[n], 0), p.n_tok); }
__device__ __forceinline__ int cu_len(const ChunkParams& p, int n) {
  const int s = cu_start(p, n);
  return min(max(p.cu[n + 1], s), p.n_tok) - s;
}
__device__ __forceinline__ int first_slot(const ChunkParams& p, int n) { return cu_start(p, n) / CH + n; }

__device__ __forceinline__ SeqRange seq_range(const ChunkParams& p, int n) {
  SeqRange r;
  if (p.cu == nullptr) {
    r.tok0 = static_cast<int64_t>(n) * p.T;
    r.len = p.T;
    r.chunk0 = n * n_chunks(p.T);
    return r;
  }
  r.tok0 = cu_start(p, n);
  r.len = cu_len(p, n);
  r.chunk0 = first_slot(p, n);
  return r;
}

// Where a chunk slot lies: its sequence, the sequence's first token and
// length, the chunk's index in it, its first token and valid length.
struct ChunkPos {
  int seq, seq_len, ci, len;
  int64_t seq_tok0, tok0;
};

// Global chunk index -> its position.  False for a slot past the end or one
// no sequence uses; then `seq`, `seq_len` and `ci` still name the sequence
// whose slots the index falls among (for packed calls).
__device__ __forceinline__ bool chunk_at(const ChunkParams& p, int c, ChunkPos& cp) {
  if (p.cu == nullptr) {
    const int cps = n_chunks(p.T);
    if (cps == 0 || c >= p.n_seqs * cps) return false;
    cp.seq = c / cps;
    cp.ci = c % cps;
    cp.seq_len = p.T;
    cp.seq_tok0 = static_cast<int64_t>(cp.seq) * p.T;
  } else {
    // the last sequence whose first slot is at or below c (first slots
    // increase with n), by bisection
    int lo = 0, hi = p.n_seqs - 1;
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (first_slot(p, mid) <= c) lo = mid;
      else hi = mid - 1;
    }
    cp.seq = lo;
    cp.seq_len = cu_len(p, lo);
    cp.ci = c - first_slot(p, lo);
    cp.seq_tok0 = cu_start(p, lo);
    if (cp.ci < 0 || cp.ci >= n_chunks(cp.seq_len)) return false;  // a slot no sequence uses
  }
  cp.tok0 = cp.seq_tok0 + static_cast<int64_t>(cp.ci) * CH;
  cp.len = min(CH, cp.seq_len - cp.ci * CH);
  return true;
}

// Writes p.order: the packed sequences by length, longest first (ties by
// index).  One workgroup: each thread ranks sequences tid, tid + 256, ...
// against all the others, whose lengths it reads from LDS (`lens`, room for
// kOrderMax).
__device__ void order_sequences(const ChunkParams& p, int* lens) {
  const int n = p.n_seqs;
  for (int i = threadIdx.x; i < n; i += blockDim.x) lens[i] = cu_len(p, i);
  __syncthreads();
  for (int i = threadIdx.x; i < n; i += blockDim.x) {
    const int li = lens[i];
    int r = 0;
    for (int m = 0; m < n; ++m) {
      const int lm = lens[m];
      r += (lm > li) || (lm == li && m < i);
    }
    p.order[r] = i;
  }
}

// ------------------------------------------------------- fused conv prologue

constexpr int KTAP = 4;  // conv taps

// The conv prologue (prologue_kernel in gdn_prologue.hip) for one lane's 8
// channels c0 .. c0+7 over the R tokens [t0, t0 + R) of a chunk, with that
// kernel's arithmetic and rounding, so q, k and v are bit-identical to its:
// with bf16 taps the conv on bf16 pairs (conv_pairs), with fp32 taps
// w[3] x_t + w[0] x_{t-3} + w[1] x_{t-2} + w[2] x_{t-1} (fused in that
// order); then o = silu(conv) and, with NORM, o * rsqrt(mean over the head of
// o^2 + eps) * post, the mean over this lane's 16-lane row (the head's 16
// lanes, in the prologue's lane order).  x runs over X = the sequence's conv
// state (3 rows; zeros without one) followed by its qkv rows.  Tokens past
// the chunk's end repeat its last row.  Every load is issued before the
// first conversion.
template <int WDT, int R, bool NORM>
__device__ __forceinline__ void conv_run(const ChunkParams& p, const ChunkPos& cp, int c0, int t0, float post,
                                         u32x4 (&out)[R]) {
  Raw8<WDT> wr[KTAP];
#pragma unroll
  for (int i = 0; i < KTAP; ++i) wr[i] = load_raw8<WDT>(p.conv_w, static_cast<int64_t>(c0) * KTAP + 8 * i);
  const int pos = cp.ci * CH + t0;  // the run's first token within its sequence
  Raw8<GDN_DTYPE_BF16> xw[KTAP - 1];
  float wm[KTAP - 1];
#pragma unroll
  for (int i = 0; i < KTAP - 1; ++i) {
    const int xi = pos + i;
    const bool from_cs = xi < KTAP - 1;
    const bool cs_row = from_cs && p.cs_in != nullptr;
    // without a conv state the row is the sequence's first qkv row, zeroed;
    // a run that starts past the chunk's end (outputs discarded) reads
    // within the chunk's valid rows
    const int tp = from_cs ? 0 : min(xi - (KTAP - 1), cp.ci * CH + cp.len - 1);
    const int64_t off = cs_row ? (static_cast<int64_t>(cp.seq) * (KTAP - 1) + xi) * p.C + c0
                               : (cp.seq_tok0 + tp) * p.qkv_ld + c0;
    xw[i] = load_raw8<GDN_DTYPE_BF16>(cs_row ? static_cast<const void*>(p.cs_in) : p.qkv, off);
    wm[i] = from_cs && !cs_row ? 0.0f : 1.0f;
  }
  Raw8<GDN_DTYPE_BF16> xs[R];
#pragma unroll
  for (int u = 0; u < R; ++u)
    xs[u] = load_raw8<GDN_DTYPE_BF16>(p.qkv, (cp.tok0 + min(t0 + u, cp.len - 1)) * p.qkv_ld + c0);
  // token u's SiLU outputs o and their sum of squares ss -> out[u]
  auto finish = [&](int u, float (&o)[CPL], float ss) {
    if constexpr (NORM) {
      ss = head_sum<16>(ss);
      const float sc = rsqrtf(ss / static_cast<float>(DK) + p.conv_eps) * post;
#pragma unroll
      for (int j = 0; j < CPL; ++j) o[j] *= sc;
    }
    out[u] = u32x4{pk_bf16(o[0], o[1]), pk_bf16(o[2], o[3]), pk_bf16(o[4], o[5]), pk_bf16(o[6], o[7])};
  };
  if constexpr (WDT == GDN_DTYPE_BF16) {
    uint32_t w01[CPL], w23[CPL];
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
      w01[j] = wr[j >> 1].v[2 * (j & 1)];
      w23[j] = wr[j >> 1].v[2 * (j & 1) + 1];
    }
    u32x4 rw[KTAP - 1];  // X_{t-3}, X_{t-2}, X_{t-1} of the current token t
#pragma unroll
    for (int i = 0; i < KTAP - 1; ++i) rw[i] = row_or_zero(wm[i] != 0.0f, xw[i].v);
    uint32_t pa[CPL], pb[CPL];  // p(t - 2), p(t - 1)
    row_pairs(rw[0], rw[1], pa);
    row_pairs(rw[1], rw[2], pb);
#pragma unroll
    for (int u = 0; u < R; ++u) {
      uint32_t pc[CPL];  // p(t)
      row_pairs(rw[KTAP - 2], xs[u].v, pc);
      float o[CPL];
      float ss = 0.0f;
#pragma unroll
      for (int j = 0; j < CPL; ++j) {
        o[j] = silu(conv_pairs(w01[j], w23[j], pa[j], pc[j]));
        ss = fmaf(o[j], o[j], ss);
      }
#pragma unroll
      for (int j = 0; j < CPL; ++j) {
        pa[j] = pb[j];
        pb[j] = pc[j];
      }
      rw[KTAP - 2] = xs[u].v;
      finish(u, o, ss);
    }
  } else {
    float w[KTAP][CPL];
    {
      float wv[CPL * KTAP];
#pragma unroll
      for (int i = 0; i < KTAP; ++i) unpack8<WDT>(wr[i], *reinterpret_cast<float(*)[CPL]>(&wv[8 * i]));
#pragma unroll
      for (int j = 0; j < CPL; ++j)
#pragma unroll
        for (int i = 0; i < KTAP; ++i) w[i][j] = wv[j * KTAP + i];
    }
    float win[KTAP - 1][CPL];
#pragma unroll
    for (int i = 0; i < KTAP - 1; ++i) {
      unpack8<GDN_DTYPE_BF16>(xw[i], win[i]);
#pragma unroll
      for (int j = 0; j < CPL; ++j) win[i][j] = wm[i] != 0.0f ? win[i][j] : 0.0f;
    }
#pragma unroll
    for (int u = 0; u < R; ++u) {
      float x[CPL], o[CPL];
      unpack8<GDN_DTYPE_BF16>(xs[u], x);
      float ss = 0.0f;
#pragma unroll
      for (int j = 0; j < CPL; ++j) {
        float acc = w[KTAP - 1][j] * x[j];
#pragma unroll
        for (int i = 0; i < KTAP - 1; ++i) acc = fmaf(w[i][j], win[i][j], acc);
        o[j] = silu(acc);
        ss = fmaf(o[j], o[j], ss);
      }
#pragma unroll
      for (int i = 0; i < KTAP - 2; ++i)
#pragma unroll
        for (int j = 0; j < CPL; ++j) win[i][j] = win[i + 1][j];
#pragma unroll
      for (int j = 0; j < CPL; ++j) win[KTAP - 2][j] = x[j];
      finish(u, o, ss);
    }
  }
}

// The new conv state of a sequence whose last chunk this workgroup holds
// (or of an empty sequence): X's last 3 rows, X[len + i], on the channels
// of this v-head and, from the k-head's first v-head, of its q and k heads.
// Thread i < 144 copies 8 channels of one row.
__device__ __forceinline__ void conv_state_rows(const ChunkParams& p, int seq, int64_t seq_tok0, int seq_len,
                                                int hk, int hv, bool first_v, int tid) {
  if (p.cs_out == nullptr || tid >= 3 * 48) return;
  const int row = tid / 48, grp = tid % 48;
  if (grp < 32 && !first_v) return;
  const int c0 = grp < 16 ? hk * DK + 8 * grp
                          : (grp < 32 ? (p.Hk + hk) * DK + 8 * (grp - 16) : 2 * p.Hk * DK + hv * DV + 8 * (grp - 32));
  const int xi = seq_len + row;
  u32x4 v = {0u, 0u, 0u, 0u};
  if (xi >= KTAP - 1) {
    v = *reinterpret_cast<const u32x4*>(p.qkv + (seq_tok0 + xi - (KTAP - 1)) * p.qkv_ld + c0);
  } else if (p.cs_in != nullptr) {
    v = *reinterpret_cast<const u32x4*>(p.cs_in + (static_cast<int64_t>(seq) * (KTAP - 1) + xi) * p.C + c0);
  }
  *reinterpret_cast<u32x4*>(p.cs_out + (static_cast<int64_t>(seq) * (KTAP - 1) + row) * p.C + c0) = v;
}

// ------------------------------------------------------------ chunk_prep

// One DPP move of a double (both 32-bit halves with the same control);
// lanes the move does not reach read 0.
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ double dpp_d(double x) {
  const uint64_t u = __builtin_bit_cast(uint64_t, x);
  const uint32_t lo = __builtin_amdgcn_update_dpp(0, static_cast<int>(u), CTRL, ROW_MASK, 0xF, false);
  const uint32_t hi = __builtin_amdgcn_update_dpp(0, static_cast<int>(u >> 32), CTRL, ROW_MASK, 0xF, false);
  return __builtin_bit_cast(double, (static_cast<uint64_t>(hi) << 32) | lo);
}

// Inclusive prefix sum of a double over the 64 lanes: row shifts by 1, 2, 4
// and 8 scan each 16-lane row, then the gfx9 row broadcasts carry the row
// totals (lane 15 of a row to the next row, for rows 1 and 3; lane 31 to
// rows 2 and 3).
__device__ __forceinline__ double wave_scan_d(double x) {
  x += dpp_d<0x111, 0xF>(x);  // row_shr:1
  x += dpp_d<0x112, 0xF>(x);  // row_shr:2
  x += dpp_d<0x114, 0xF>(x);  // row_shr:4
  x += dpp_d<0x118, 0xF>(x);  // row_shr:8
  x += dpp_d<0x142, 0xA>(x);  // row_bcast:15
  x += dpp_d<0x143, 0xC>(x);  // row_bcast:31
  return x;
}

// KT_LDS: the scan forms K^T from K in LDS, so the record carries no K^T.
// Four workgroups per CU: 35.6 KB of LDS each and at most 128 VGPRs (four
// waves per SIMD; left to itself the compiler takes 137-138, which leaves
// three).  At 4096 tokens x 32 heads the 2048 workgroups then run in two
// full rounds instead of two and two thirds.
//
// CONV (1: bf16 taps, 2: fp32 taps): the conv prologue is fused in.  The
// workgroup forms its chunk's q and k rows (its k-head) and v rows (its
// v-head) from the qkv rows with the conv prologue's arithmetic, writes v
// for the scan and, at a sequence's last chunk, the new conv state; the
// slot of an empty packed sequence passes its conv state through.
//
// MASK: a token mask is given (the unmasked kernels carry none of its code).
template <bool KT_LDS, int CONV, bool MASK>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(4))) void chunk_prep_kernel(const ChunkParams p) {
  // Two 17 KB buffers, each reused once (LDS stays under 40 KB, so four
  // workgroups fit on a CU):  buf0 = K rows, then A;  buf1 = Q rows, then
  // the P hi/lo planes in fragment order, then (I + A)^{-1}.  The extra last
  // workgroup of a packed call orders the sequences in buf0 instead.
  constexpr int kBuf = CH * KP * 2;
  static_assert(kBuf == CH * (CH + 4) * 4, "A and T must fill the K / Q buffers exactly");
  static_assert(kBuf >= 2 * CH * CH * 2, "P staging must fit in the Q buffer");
  static_assert(kBuf >= kOrderMax * 4, "the sequence lengths must fit in buf0");
  __shared__ __align__(16) unsigned char buf0[kBuf];
  __shared__ __align__(16) unsigned char buf1[kBuf];
  if (p.order != nullptr && blockIdx.x == gridDim.x - 1) {
    order_sequences(p, reinterpret_cast<int*>(buf0));
    return;
  }
  // work index = chunk * Hv + hv: both v-heads of a k-head (GQA) share an XCD
  const int w = xcd_work_index(gridDim.x - (p.order != nullptr ? 1 : 0));
  const int c = w / p.Hv;
  const int hv = w % p.Hv;
  const int hk = hv / p.group;
  const bool first_v = hv % p.group == 0;  // writes the k-head's K^T, K and Q
  ChunkPos cp;
  if (!chunk_at(p, c, cp)) {
    if constexpr (CONV != 0) {
      if (p.cu != nullptr && cp.seq_len == 0 && cp.ci == 0)
        conv_state_rows(p, cp.seq, cp.seq_tok0, 0, hk, hv, first_v, threadIdx.x);
    }
    return;
  }
  const int64_t tok0 = cp.tok0;
  const int len = cp.len;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform
  const int lr = lane & 15, lq = lane >> 4, lg8 = lq * 8;

  __shared__ __align__(16) double Ld[CH];  // L_t log2(e) (the decays' exponents, base 2)
  __shared__ float Bs[CH];
  __shared__ float Ys[MASK ? CH : 1];  // 1, or 0 at a masked token (its row of P is zero)
  auto Ks = reinterpret_cast<uint16_t(*)[KP]>(buf0);
  auto Qs = reinterpret_cast<uint16_t(*)[KP]>(buf1);
  auto As = reinterpret_cast<float(*)[CH + 4]>(buf0);
  auto Ti = reinterpret_cast<float(*)[CH + 4]>(buf1);
  uint16_t* Pst = reinterpret_cast<uint16_t*>(buf1);

  // Gate loads first, raw (wave 0 uses them; every wave issues them, so no
  // branch lets the compiler start converting them early, which would wait),
  // so waiting for them does not wait for the K/Q rows queued behind; then
  // the rows (rows past the chunk's end read its last row and are zeroed at
  // the LDS store); the gate transforms only after every load is issued.
  const GateRaw gr = load_gate_raw(p.ga, (tok0 + min(lane, len - 1)) * p.ga.ld + hv, hv);
  const uint8_t mk = MASK ? *(gbl_u8*)(p.mask + tok0 + min(lane, len - 1)) : 1;
  double L_lane = 0.0;  // wave 0: L_t of token `lane` (its record entries are written last)
  float b_lane = 0.0f;
  bool on_lane = false;  // wave 0: token `lane` is real and not masked
  asm volatile("" ::: "memory");  // keeps the gate loads issued ahead of the rows
  u32x4 kr[4], qr[4];
  bool kq_on[4];  // the row is a real token (and, with MASK, not masked)
  if constexpr (CONV == 0) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int i = tid + 256 * j;
      const int r = i / (DK / 8), cc = (i % (DK / 8)) * 8;
      const int64_t off = ((tok0 + min(r, len - 1)) * p.Hk + hk) * DK + cc;
      kr[j] = *reinterpret_cast<const u32x4*>(p.k + off);
      qr[j] = *reinterpret_cast<const u32x4*>(p.q + off);
      // a masked token's k and q rows are zeros, as the reference's where()
      // keeps whatever they hold out of the state: they then add nothing to
      // any other token's A, P, X or state update (beta = 0 alone would
      // still let a non-finite value through as 0 * inf)
      kq_on[j] = r < len && (!MASK || *(gbl_u8*)(p.mask + tok0 + min(r, len - 1)) != 0);
    }
  }
  unsigned char* rec = p.ws + (static_cast<size_t>(c) * p.Hv + hv) * kRecBytes;
  if (wave == 0) {
    float lg, bt;
    log_gates(p.ga, gr, lg, bt);
    // padding and masked tokens: no decay, no write (a masked token keeps
    // the state and its y is 0); g = 0 (pre-transformed) stays finite
    on_lane = lane < len && mk != 0;
    lg = on_lane ? fmaxf(lg, -1.0e30f) : 0.0f;
    bt = on_lane ? bt : 0.0f;
    L_lane = wave_scan_d(lg);
    Ld[lane] = L_lane * kLog2e;
    Bs[lane] = bt;
    if constexpr (MASK) Ys[lane] = on_lane ? 1.0f : 0.0f;
    b_lane = bt;
  }
  if constexpr (CONV == 0) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int i = tid + 256 * j;
      const int r = i / (DK / 8), cc = (i % (DK / 8)) * 8;
      const u32x4 kv = row_or_zero(kq_on[j], kr[j]), qv = row_or_zero(kq_on[j], qr[j]);
      *reinterpret_cast<u32x4*>(&Ks[r][cc]) = kv;
      *reinterpret_cast<u32x4*>(&Qs[r][cc]) = qv;
      if (first_v) {
        *reinterpret_cast<u32x4*>(reinterpret_cast<uint16_t*>(rec + kOffKf) + frag_elem(r, cc, DK / 32)) = kv;
        *reinterpret_cast<u32x4*>(reinterpret_cast<uint16_t*>(rec + kOffQf) + frag_elem(r, cc, DK / 32)) = qv;
      }
    }
  } else {
    // 16-lane row rw of the workgroup takes 4 tokens, [4 rw, 4 rw + 4), of
    // one head, lane g of the row channels 8 g .. 8 g + 7 of it: q, then k
    // (to LDS and the records, as the loads above would), then v (for the
    // scan).
    constexpr int WDT = CONV == 2 ? GDN_DTYPE_F32 : GDN_DTYPE_BF16;
    const int rw = 4 * wave + lq, g = lr, t0 = 4 * rw;
#pragma unroll
    for (int role = 0; role < 2; ++role) {
      u32x4 o[4];
      const float post = role == 0 ? 1.0f / static_cast<float>(DK) : rsqrtf(static_cast<float>(DK));
      conv_run<WDT, 4, true>(p, cp, (role * p.Hk + hk) * DK + 8 * g, t0, post, o);
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int r = t0 + u;
        const u32x4 val = row_or_zero(r < len, o[u]);
        *reinterpret_cast<u32x4*>(role == 0 ? &Qs[r][8 * g] : &Ks[r][8 * g]) = val;
        if (first_v)
          *reinterpret_cast<u32x4*>(reinterpret_cast<uint16_t*>(rec + (role == 0 ? kOffQf : kOffKf)) +
                                    frag_elem(r, 8 * g, DK / 32)) = val;
      }
    }
    {
      u32x4 o[4];
      conv_run<WDT, 4, false>(p, cp, 2 * p.Hk * DK + hv * DV + 8 * g, t0, 1.0f, o);
#pragma unroll
      for (int u = 0; u < 4; ++u)
        if (t0 + u < len)
          *reinterpret_cast<u32x4*>(p.v_out + ((tok0 + t0 + u) * p.Hv + hv) * DV + 8 * g) = o[u];
    }
    if (cp.ci == n_chunks(cp.seq_len) - 1)
      conv_state_rows(p, cp.seq, cp.seq_tok0, cp.seq_len, hk, hv, first_v, tid);
  }
  __syncthreads();

  // K K^T and Q K^T: wave w computes row block w (16 rows) x 4 column
  // blocks, as the transposed products K_j K_w^T and K_j Q_w^T (an A and a
  // B fragment have the same layout, so the operands swap roles): lane
  // (r, q) of tile j then holds row 16w + r, columns 16j + 4q .. +3 (K K^T is
  // symmetric) -- four consecutive columns of one row, which go to LDS as
  // one 16-byte (A) or 8-byte (P hi, P lo) store.
  f32x4 kk[4], qk[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    kk[j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    qk[j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  }
  // K^T for the scan's state update, as MFMA A-fragments (rows dk, columns
  // tokens): a product with a one-hot B turns this wave's K rows into 16x16
  // tiles whose lane (r, q) holds K[16w + 4q .. +3][16d + r], i.e. 4
  // consecutive tokens of one dk -- half of the 16 bytes of fragment lane
  // r + 16 * (2 * (w % 2) + q / 2).  Written once per k-head (by its first
  // v-head), 8 bytes per lane and tile.
  bf16x8 eye[2];
#pragma unroll
  for (int h = 0; h < 2; ++h)
#pragma unroll
    for (int e = 0; e < 8; ++e) eye[h][e] = static_cast<__bf16>(lg8 + e == lr + 16 * h ? 1.0f : 0.0f);
  unsigned char* KTg = rec + kOffKT + (wave >> 1) * 1024 + (lr + 16 * (2 * (wave & 1) + (lq >> 1))) * 16 + (lq & 1) * 8;
#pragma unroll
  for (int s = 0; s < DK / 32; ++s) {
    const int kc = s * 32 + lg8;
    const bf16x8 ak = lds8(&Ks[16 * wave + lr][kc]);
    const bf16x8 aq = lds8(&Qs[16 * wave + lr][kc]);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const bf16x8 bk = lds8(&Ks[16 * j + lr][kc]);
      kk[j] = mfma16(bk, ak, kk[j]);
      qk[j] = mfma16(bk, aq, qk[j]);
    }
    if (!KT_LDS && first_v) {
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const f32x4 t = mfma16(ak, eye[h], f32x4{0.0f, 0.0f, 0.0f, 0.0f});
        // dk block d = 2s + h: fragment (d, token column wave / 2) at 2 KB * d
        *reinterpret_cast<u32x2*>(KTg + (2 * s + h) * 2048) = u32x2{pk_bf16(t[0], t[1]), pk_bf16(t[2], t[3])};
      }
    }
  }
  // every wave has its K K^T / Q K^T products in registers; K and Q in LDS
  // are no longer read, so their buffers take A and the P planes
  __syncthreads();

  // Decays, A (to LDS, fp32) and P (hi/lo bf16, staged in fragment order):
  // lane (r, q) takes row t = 16w + r, columns 16j + 4q .. +3.
  {
    const int t = 16 * wave + lr;
    typedef double f64x2 __attribute__((ext_vector_type(2)));
    const double Lt = Ld[t];
    const float bt = Bs[t];
    const float yt = MASK ? Ys[t] : 1.0f;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int c0 = 16 * j + 4 * lq;
      const f64x2 l01 = *reinterpret_cast<const f64x2*>(&Ld[c0]);  // two 16-byte reads for four columns
      const f64x2 l23 = *reinterpret_cast<const f64x2*>(&Ld[c0 + 2]);
      const double Lc[4] = {l01.x, l01.y, l23.x, l23.y};
      f32x4 av;
      float pv[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int col = c0 + i;
        const float dec = col <= t ? __builtin_amdgcn_exp2f(static_cast<float>(Lt - Lc[i])) : 0.0f;
        av[i] = col < t ? bt * dec * kk[j][i] : 0.0f;
        pv[i] = MASK ? (dec * qk[j][i]) * yt : dec * qk[j][i];
      }
      *reinterpret_cast<f32x4*>(&As[t][c0]) = av;
      split4_store(f32x4{pv[0], pv[1], pv[2], pv[3]}, Pst + frag_elem(t, c0, CH / 32),
                   Pst + CH * CH + frag_elem(t, c0, CH / 32));
    }
  }
  __syncthreads();

  // (I + A)^{-1}, A strictly lower.  Its diagonal 16x16 blocks by forward
  // substitution (wave 0, one lane per (block, column)), into registers --
  // only A is read -- while waves 1-3 copy the P planes out of the buffer the
  // inverse takes next: a linear 16 KB copy (hi then lo, as in the record).
  // The P fragments above the diagonal that hold only zeros -- row blocks 0
  // and 1, column block 1 (fragments 1 and 3 of a plane) -- are not written:
  // the scan never reads them.
  const int dbase = 16 * (lane >> 4), dcol = lane & 15;
  float x[16];
  if (wave == 0) {
    float a[16][16];
#pragma unroll
    for (int t = 1; t < 16; ++t)
#pragma unroll
      for (int i = 0; i < t; ++i) a[t][i] = As[dbase + t][dbase + i];
#pragma unroll
    for (int t = 0; t < 16; ++t) {
      float acc = t == dcol ? 1.0f : 0.0f;
#pragma unroll
      for (int i = 0; i < t; ++i) acc = fmaf(-a[t][i], x[i], acc);
      x[t] = t < dcol ? 0.0f : acc;
    }
  } else {
    for (int i = tid - 64; i < 1024; i += 192) {
      const int frag = (i & 511) >> 6;
      if (frag != 1 && frag != 3)
        *reinterpret_cast<u32x4*>(rec + kOffPh + 16 * i) = *reinterpret_cast<const u32x4*>(Pst + 8 * i);
    }
  }
  __syncthreads();  // the P planes are out: their buffer takes (I + A)^{-1}
  if (wave == 0) {
#pragma unroll
    for (int t = 0; t < 16; ++t) Ti[dbase + t][dbase + dcol] = x[t];
  }
  __syncthreads();
  // Off-diagonal blocks.  Block (I, J) belongs to wave J, which forms its
  // column of blocks top-down:
  //   M = sum_{K=J}^{I-1} A_IK T_KJ,   T_IJ = -T_II M
  // Each 16x16x16 block product is four fp32 MFMAs (16x16x4), with the k
  // index of step s and lane l taken as 4 (l / 16) + s: lane l then supplies
  // A[l % 16][4 (l / 16) .. +3] (one 16-byte read of a row) and
  // B[4 (l / 16) .. +3][l % 16] -- which is what the lane holds of an
  // accumulator tile (rows 4 (l / 16) .. +3 of column l % 16).  So M feeds
  // the second product, and the wave's earlier blocks T_KJ (K > J) the
  // first, straight from registers; only A, T_JJ and T_II come from LDS, and
  // no wave reads another's off-diagonal blocks until the barrier below.
  {
    const int ln = lane & 15, lk = lane >> 4;
    const int J = wave;
    f32x4 tcol[3];  // T_{J+1,J} .. T_{J+3,J}
    float tjj[4];
#pragma unroll
    for (int s4 = 0; s4 < 4; ++s4) tjj[s4] = Ti[16 * J + 4 * lk + s4][16 * J + ln];
#pragma unroll
    for (int d = 1; d < 4; ++d) {
      const int I = J + d;
      if (I < 4) {  // wave-uniform
        f32x4 m = {0.0f, 0.0f, 0.0f, 0.0f};
        {
          const f32x4 a4 = *reinterpret_cast<const f32x4*>(&As[16 * I + ln][16 * J + 4 * lk]);
#pragma unroll
          for (int s4 = 0; s4 < 4; ++s4) m = __builtin_amdgcn_mfma_f32_16x16x4f32(a4[s4], tjj[s4], m, 0, 0, 0);
        }
#pragma unroll
        for (int e = 0; e < 2; ++e) {
          const int Kb = J + 1 + e;
          if (e < d - 1) {
            const f32x4 a4 = *reinterpret_cast<const f32x4*>(&As[16 * I + ln][16 * Kb + 4 * lk]);
#pragma unroll
            for (int s4 = 0; s4 < 4; ++s4) m = __builtin_amdgcn_mfma_f32_16x16x4f32(a4[s4], tcol[e][s4], m, 0, 0, 0);
          }
        }
        const f32x4 tii = *reinterpret_cast<const f32x4*>(&Ti[16 * I + ln][16 * I + 4 * lk]);
        f32x4 tv = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int s4 = 0; s4 < 4; ++s4) tv = __builtin_amdgcn_mfma_f32_16x16x4f32(tii[s4], m[s4], tv, 0, 0, 0);
        tv = -tv;
        tcol[d - 1] = tv;
#pragma unroll
        for (int i = 0; i < 4; ++i) Ti[16 * I + 4 * lk + i][16 * J + ln] = tv[i];
      }
    }
  }
  __syncthreads();  // every block of (I + A)^{-1} is in LDS
  uint16_t* Th = reinterpret_cast<uint16_t*>(rec + kOffTh);
  uint16_t* Tl = reinterpret_cast<uint16_t*>(rec + kOffTl);
  // one 16-byte group (8 columns of a row) per thread and pass; blocks
  // above the diagonal are zero (never written in Ti), and the all-zero
  // fragments (rows < 32, columns >= 32) are not stored, as for P
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int i = tid + 256 * j;
    const int r = i >> 3, cc = (i & 7) * 8;
    if (r < 32 && cc >= 32) continue;
    const bool upper = (cc >> 4) > (r >> 4);
    const f32x4 z = {0.0f, 0.0f, 0.0f, 0.0f};
    const f32x4 a = upper ? z : *reinterpret_cast<const f32x4*>(&Ti[r][cc]);
    const f32x4 b = upper ? z : *reinterpret_cast<const f32x4*>(&Ti[r][cc + 4]);
    split4_store(a, Th + frag_elem(r, cc, CH / 32), Tl + frag_elem(r, cc, CH / 32));
    split4_store(b, Th + frag_elem(r, cc + 4, CH / 32), Tl + frag_elem(r, cc + 4, CH / 32));
  }
  // the gates' record entries (only the scan reads them)
  if (wave == 0) {
    const uint64_t u = __builtin_bit_cast(uint64_t, L_lane);
    const uint32_t lo = __builtin_amdgcn_readlane(static_cast<int>(u), 63);
    const uint32_t hi = __builtin_amdgcn_readlane(static_cast<int>(u >> 32), 63);
    const double LC = __builtin_bit_cast(double, (static_cast<uint64_t>(hi) << 32) | lo);
    reinterpret_cast<float*>(rec + kOffGam)[lane] = expf(static_cast<float>(L_lane));
    reinterpret_cast<float*>(rec + kOffE)[lane] = expf(static_cast<float>(LC - L_lane));
    reinterpret_cast<float*>(rec + kOffBeta)[lane] = b_lane;
    reinterpret_cast<float*>(rec + kOffGy)[lane] = on_lane ? expf(static_cast<float>(L_lane)) : 0.0f;
  }
}

// ------------------------------------------------------------ chunk_scan
//
// One workgroup (4 waves) owns a 16-row tile of one head's state and walks
// that head's chunks.  Wave w produces the chunk's quantities for tokens
// [16w, 16w+16) (X_K, X_Q, R, U, Y) and updates state columns
// [32w, 32w+32).  Every MFMA operand that is specific to a wave -- its K, Q,
// T and P rows, its K^T rows (or, with several workgroups per CU, K rows
// read back transposed from LDS) and its V values -- is loaded from global
// memory straight into registers in MFMA layout, and reloaded for the next
// chunk right after its last use, so those loads overlap the rest of the
// chunk.  Otherwise LDS carries what the waves exchange -- the state (hi/lo
// bf16) and R^T, U^T, (eU)^T, three barriers per chunk -- and the chunk's
// per-token gates, loaded once a chunk.
//
// The state update and Y are computed transposed (S^T += K^T (eU),
// Y^T = gamma X_Q^T + U^T P^T): a lane then holds 4 consecutive state
// columns / value channels, so the state goes to LDS and y to memory in
// 8-byte stores.  Global operands are read through buffer descriptors
// rebased per chunk (scalar work) with loop-invariant lane offsets; a
// descriptor's extent ends at the chunk's last token, so the hardware returns
// zeros for the padding rows of a short chunk and drops their y stores.

typedef __amdgpu_buffer_rsrc_t BufRsrc;

constexpr int kBufFlags = 0x00020000;  // raw buffer, 32-bit data format (gfx9)

__device__ __forceinline__ BufRsrc buf_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, static_cast<int>(bytes), kBufFlags);
}

__device__ __forceinline__ bf16x8 buf_bf16x8(BufRsrc r, uint32_t voff, int soff) {
  return __builtin_bit_cast(bf16x8, __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0));
}

__device__ __forceinline__ f32x4 buf_f32x4(BufRsrc r, uint32_t voff) {
  return __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(r, voff, 0, 0));
}

// One wave's operands of one chunk (all in MFMA operand layouts).
struct WaveOps {
  bf16x8 k[4], q[4];     // K / Q rows 16w + lr, columns 32s + 8lq ..
  bf16x8 th[2], tl[2];   // T rows 16w + lr, columns 32s + 8lq .. (hi / lo)
  bf16x8 ph[2], pl[2];   // P rows, same layout
  bf16x8 kt[2][2];       // K^T rows 32w + 16j + lr, columns 32s + 8lq ..
  uint16_t v[2][4];      // V[16w + 4lq + i][dv0 + 16t + lr] (bf16 bits) of tile t
  f32x4 g, b, e;         // gamma / beta / e of tokens 16w + 4lq + i
  float gl;              // the next chunk's gate value of this lane, until it goes to LDS
  float gC;              // gamma of the chunk's last token
};

// A chunk's descriptors: V and Y (this v-head, from state row dv0) and all
// v-heads' workspace records of the chunk.
struct ChunkBufs {
  BufRsrc v, y, rec;
  const float* gam;      // gamma of this head's record
};

constexpr int kTiles = DV / DVT;  // state-row tiles per head (8)
constexpr int kXcds = 8;
constexpr int kCUs = 256;  // compute units of an MI355X (8 XCDs x 32)

// KT_LDS: K^T comes from transposed LDS reads of the K rows the waves hold
// (the record's K^T is then not written or read).  That trades 16 KB of
// operand loads per chunk for 16 KB of LDS writes and reads: it pays when
// several workgroups share a CU, and costs a little on the chain when one
// workgroup has the CU to itself.
// TPW: 16-row state tiles per workgroup.  With two, every operand a wave
// loads (K, Q, T, P, K^T, gates) serves 32 state rows: half the operand
// bytes per row, for a longer chain per chunk (twice the MFMAs and LDS
// exchanges per wave).  It pays when the tiles outnumber the CUs and the
// operand traffic, not one long chain, bounds the scan.
// MASK: a token mask was given.  A masked token has beta = 0, and its R is
// then taken as 0 outright, so a non-finite v there stays out of U (the
// prep zeroes its k and q rows likewise).
template <bool KT_LDS, int TPW, bool MASK>
__global__ __launch_bounds__(256) void chunk_scan_kernel(const ChunkParams p) {
  // Block b runs on XCD b % 8.  The v-heads of one k-head (a GQA group,
  // which share its K, Q and K^T) form a unit; units (over all sequences,
  // longest sequence first) are dealt to XCDs round-robin, and the 8 tiles of
  // each head go to the unit's XCD, where they share its operands in L2.
  const int blk = blockIdx.x;
  const int xcd = blk % kXcds, r8 = blk / kXcds;
  constexpr int kWgs = kTiles / TPW;  // workgroups per head
  const int tile = r8 % kWgs;
  const int slot_x = r8 / kWgs;  // head slot on this XCD
  const int head_rank = ((slot_x / p.group) * kXcds + xcd) * p.group + slot_x % p.group;
  if (head_rank >= p.n_seqs * p.Hv) return;
  const int seq = p.order != nullptr ? p.order[head_rank / p.Hv] : head_rank / p.Hv;
  int slot = seq;
  if (p.state_index != nullptr) {
    slot = p.state_index[seq];
    if (slot < 0 || slot >= p.n_slots) return;  // uniform, before any barrier
  }
  const int hv = head_rank % p.Hv;
  const int dv0 = tile * DVT * TPW;
  const int hk = hv / p.group;
  const int hv_k = hk * p.group;  // the v-head whose record holds this k-head's K^T
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lr = lane & 15, lq = lane >> 4, lg8 = lq * 8;
  const SeqRange sr = seq_range(p, seq);
  const int nch = n_chunks(sr.len);

  constexpr int NR = DVT * TPW;  // state rows of this workgroup; tile t holds rows 16t ..
  __shared__ __align__(16) uint16_t Sh[NR][KP], Sl[NR][KP];  // S0 [row][dk], hi / lo
  __shared__ __align__(16) uint16_t Rh[NR][CP], Rl[NR][CP];  // R^T [row][token]
  __shared__ __align__(16) uint16_t Uh[NR][CP], Ul[NR][CP];  // U^T
  __shared__ __align__(16) uint16_t Eh[NR][CP], El[NR][CP];  // (diag(e) U)^T
  __shared__ __align__(16) uint16_t Kl[KT_LDS ? CH : 1][KP];   // K [token][dk] (KT_LDS)
  __shared__ __align__(16) float Gs[4][CH];  // gamma, e, beta and the y gamma of the chunk

  // Loop-invariant lane offsets (bytes) into the per-chunk descriptors:
  // fragment (rb, cb) of a record matrix is 1 KB at (rb * n_cb + cb) KB.
  const uint32_t hv_row = static_cast<uint32_t>(p.Hv) * DV * 2;
  const uint32_t rec_hk = static_cast<uint32_t>(hv_k) * kRecBytes;
  const uint32_t off_kq = rec_hk + kOffKf + (4 * wave * 64 + lane) * 16;  // K (+ Q plane)
  uint32_t off_v[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) off_v[i] = (16 * wave + 4 * lq + i) * hv_row + 2 * lr;
  const uint32_t off_y = (16 * wave + lr) * hv_row + 8 * lq;
  const uint32_t rec_hv = static_cast<uint32_t>(hv) * kRecBytes;
  const uint32_t off_rows = rec_hv + (2 * wave * 64 + lane) * 16;        // T, P rows 16w + lr
  const uint32_t off_kt = rec_hk + kOffKT + (4 * wave * 64 + lane) * 16;  // K^T rows 32w + 16j + lr
  // a lane loads array lq (gamma, e, beta, y gamma) of token 16w + lr
  const uint32_t off_gl = rec_hv + (lq == 3 ? kOffGy : kOffGam + lq * CH * 4) + (16 * wave + lr) * 4;

  // Bases of the chunk whose descriptors come next, advanced by one chunk at
  // a time (a 64-bit add each) rather than recomputed from the chunk index.
  const size_t vy_step = static_cast<size_t>(CH) * hv_row;
  const size_t rec_step = static_cast<size_t>(p.Hv) * kRecBytes;
  const unsigned char* vb = reinterpret_cast<const unsigned char*>(p.v + (sr.tok0 * p.Hv + hv) * DV + dv0);
  const unsigned char* yb = reinterpret_cast<const unsigned char*>(p.y + (sr.tok0 * p.Hv + hv) * DV + dv0);
  const unsigned char* rb = p.ws + static_cast<size_t>(sr.chunk0) * rec_step;
  int left = sr.len;  // tokens from the chunk at vb to the sequence's end
  auto bufs_here = [&]() {
    const uint32_t last = static_cast<uint32_t>(min(CH, left) - 1);
    ChunkBufs c;
    c.v = buf_rsrc(vb, last * hv_row + DV * 2);
    c.y = buf_rsrc(yb, last * hv_row + DV * 2);
    c.rec = buf_rsrc(rb, static_cast<uint32_t>(rec_step));
    c.gam = reinterpret_cast<const float*>(rb + rec_hv + kOffGam);
    return c;
  };
  auto advance = [&]() {
    vb += vy_step;
    yb += vy_step;
    rb += rec_step;
    left -= CH;
  };

  WaveOps o = {};
  auto load_kq = [&](const ChunkBufs& c) {
    static_for<4>([&](auto s) {
      o.k[s.value] = buf_bf16x8(c.rec, off_kq + 1024 * s.value, 0);
      o.q[s.value] = buf_bf16x8(c.rec, off_kq + 1024 * s.value, kOffQf - kOffKf);
    });
  };
  auto load_vg = [&](const ChunkBufs& c) {
    static_for<TPW>([&](auto t) {
      static_for<4>([&](auto i) {
        o.v[t.value][i.value] = __builtin_amdgcn_raw_buffer_load_b16(c.v, off_v[i.value] + 32 * t.value, 0, 0);
      });
    });
    o.gl = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(c.rec, off_gl, 0, 0));
  };
  // The per-token gates (gamma, e, beta, the y gamma) go through LDS.  Each
  // wave loads its 16 tokens' four values (one dword a lane) and stores them
  // at the end of the chunk before; every lane reads its values right after
  // the chunk's first barrier, where their latency hides behind X_K (read at
  // the stages that use them, they cost the chain more).  So every read of
  // the buffer is done before the chunk's second barrier, long before the
  // next store.  Loaded as 16-byte vectors per lane instead, every value
  // would cross the texture path 16 times; one value a lane with quad
  // broadcasts for the other three put DPP moves on the chain.
  auto store_gates = [&]() { Gs[lq][16 * wave + lr] = o.gl; };
  auto gate4 = [&](int a) { return *reinterpret_cast<const f32x4*>(&Gs[a][16 * wave + 4 * lq]); };
  // T and P are lower triangular: the rows of waves 0 and 1 (tokens < 32)
  // have no entries in the second 32-column block, whose loads and products
  // those waves skip (wave-uniform branches; the prep does not write those
  // fragments).
  const bool full_rows = wave >= 2;
  auto load_t = [&](const ChunkBufs& c) {
    static_for<2>([&](auto s) {
      if (s.value == 0 || full_rows) {
        o.th[s.value] = buf_bf16x8(c.rec, off_rows + 1024 * s.value, kOffTh);
        o.tl[s.value] = buf_bf16x8(c.rec, off_rows + 1024 * s.value, kOffTl);
      }
    });
  };
  auto tok4 = [&](const f32x4& x, auto i) { return x[i.value]; };
  auto load_kt = [&](const ChunkBufs& c) {
    if constexpr (!KT_LDS) {
      static_for<2>([&](auto j) {
        static_for<2>([&](auto s) {
          o.kt[j.value][s.value] = buf_bf16x8(c.rec, off_kt + 2048 * j.value + 1024 * s.value, 0);
        });
      });
    }
    o.gC = c.gam[CH - 1];
  };
  auto load_p = [&](const ChunkBufs& c) {
    static_for<2>([&](auto s) {
      if (s.value == 0 || full_rows) {
        o.ph[s.value] = buf_bf16x8(c.rec, off_rows + 1024 * s.value, kOffPh);
        o.pl[s.value] = buf_bf16x8(c.rec, off_rows + 1024 * s.value, kOffPl);
      }
    });
  };

  // This wave's 32 x 16 slices of S^T, one per tile t: state columns
  // [32w, 32w+32) as two 16x16 accumulator tiles; lane holds
  // S^T[32w + 16j + 4lq + i][lr], i.e. 4 consecutive columns of state row
  // dv0 + 16t + lr.
  const int64_t srow = (static_cast<int64_t>(slot) * p.Hv + hv) * DV + dv0 + lr;
  f32x4 sacc[TPW][2];
#pragma unroll
  for (int t = 0; t < TPW; ++t)
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int64_t idx = (srow + 16 * t) * DK + 32 * wave + 16 * j + 4 * lq;
      sacc[t][j] =
          p.state_in != nullptr ? *reinterpret_cast<const f32x4*>(p.state_in + idx) : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    }
  auto write_state = [&]() {
#pragma unroll
    for (int t = 0; t < TPW; ++t)
#pragma unroll
      for (int j = 0; j < 2; ++j)
        split4_store(sacc[t][j], &Sh[16 * t + lr][32 * wave + 16 * j + 4 * lq],
                     &Sl[16 * t + lr][32 * wave + 16 * j + 4 * lq]);
  };

  const ChunkBufs c0 = bufs_here();  // chunk 0 (only used when the sequence has chunks)
  if (nch > 0) {
    load_kq(c0);
    load_vg(c0);
    load_t(c0);
    load_kt(c0);
    load_p(c0);
  }
  write_state();
  store_gates();
  const f32x4 z = {0.0f, 0.0f, 0.0f, 0.0f};

  BufRsrc y_cur = c0.y;
  for (int ci = 0; ci < nch; ++ci) {
    // the next chunk's operands (the last chunk reloads its own: no branches
    // around the loads, so their waits are not forced early)
    if (ci + 1 < nch) advance();
    const ChunkBufs cn = bufs_here();
    __syncthreads();  // state hi/lo and gates of this chunk are in LDS
    o.g = gate4(0);
    o.e = gate4(1);
    o.b = gate4(2);
    const float gy = Gs[3][16 * wave + lr];

    // ---- X_K = K S0^T (tokens x rows) and X_Q^T = S0 Q^T (rows x tokens)
    f32x4 xk0[TPW], xk1[TPW], xq0[TPW], xq1[TPW];
#pragma unroll
    for (int t = 0; t < TPW; ++t) xk0[t] = xk1[t] = xq0[t] = xq1[t] = z;
    static_for<4>([&](auto s) {
      const int kc = 32 * s.value + lg8;
      static_for<TPW>([&](auto t) {
        const bf16x8 sh = lds8(&Sh[16 * t.value + lr][kc]);
        const bf16x8 sl = lds8(&Sl[16 * t.value + lr][kc]);
        xk0[t.value] = mfma16(o.k[s.value], sh, xk0[t.value]);
        xk1[t.value] = mfma16(o.k[s.value], sl, xk1[t.value]);
        xq0[t.value] = mfma16(sh, o.q[s.value], xq0[t.value]);
        xq1[t.value] = mfma16(sl, o.q[s.value], xq1[t.value]);
      });
    });
    if constexpr (KT_LDS) {
      // this wave's K rows to LDS (read transposed after the next barrier),
      // before their registers take the next chunk's K
      static_for<4>([&](auto s) {
        *reinterpret_cast<bf16x8*>(&Kl[16 * wave + lr][32 * s.value + lg8]) = o.k[s.value];
      });
    }
    load_kq(cn);

    // ---- R = beta (V - gamma X_K) -> R^T
    static_for<TPW>([&](auto t) {
      f32x4 r;
      static_for<4>([&](auto i) {
        r[i.value] = tok4(o.b, i) * (bf16_to_f32(o.v[t.value][i.value]) -
                                     tok4(o.g, i) * (xk0[t.value][i.value] + xk1[t.value][i.value]));
        if constexpr (MASK) r[i.value] = tok4(o.b, i) != 0.0f ? r[i.value] : 0.0f;
      });
      split4_store(r, &Rh[16 * t.value + lr][16 * wave + 4 * lq], &Rl[16 * t.value + lr][16 * wave + 4 * lq]);
    });
    load_vg(cn);
    __syncthreads();  // R^T complete

    // K^T fragments of this wave's state columns (KT_LDS: from the K rows in
    // LDS since the barrier above, read here so their latency is off the update)
    bf16x8 kt[2][2];
    static_for<2>([&](auto j) {
      static_for<2>([&](auto s) {
        if constexpr (KT_LDS)
          kt[j.value][s.value] =
              kt_frag(&Kl[32 * s.value + 8 * lq + (lr >> 2)][32 * wave + 16 * j.value + 4 * (lr & 3)]);
        else
          kt[j.value][s.value] = o.kt[j.value][s.value];
      });
    });

    // ---- U = T R for this wave's 16 tokens
    f32x4 u0[TPW], u1[TPW];
#pragma unroll
    for (int t = 0; t < TPW; ++t) u0[t] = u1[t] = z;
    static_for<2>([&](auto s) {
      if (s.value == 1 && !full_rows) return;
      const int kc = 32 * s.value + lg8;
      static_for<TPW>([&](auto t) {
        const bf16x8 rh = lds8(&Rh[16 * t.value + lr][kc]);
        u0[t.value] = mfma16(o.th[s.value], rh, u0[t.value]);
        u1[t.value] = mfma16(o.th[s.value], lds8(&Rl[16 * t.value + lr][kc]), u1[t.value]);
        u1[t.value] = mfma16(o.tl[s.value], rh, u1[t.value]);
      });
    });
    load_t(cn);
    {
      const f32x4 ev = {tok4(o.e, std::integral_constant<int, 0>{}), tok4(o.e, std::integral_constant<int, 1>{}),
                        tok4(o.e, std::integral_constant<int, 2>{}), tok4(o.e, std::integral_constant<int, 3>{})};
      static_for<TPW>([&](auto t) {
        const f32x4 uv = u0[t.value] + u1[t.value];
        split4_store(uv, &Uh[16 * t.value + lr][16 * wave + 4 * lq], &Ul[16 * t.value + lr][16 * wave + 4 * lq]);
        split4_store(ev * uv, &Eh[16 * t.value + lr][16 * wave + 4 * lq], &El[16 * t.value + lr][16 * wave + 4 * lq]);
      });
    }
    __syncthreads();  // U^T, (eU)^T complete

    // ---- S^T = gamma_C S0^T + K^T (diag(e) U) on this wave's 32 columns
#pragma unroll
    for (int t = 0; t < TPW; ++t)
#pragma unroll
      for (int j = 0; j < 2; ++j) sacc[t][j] *= o.gC;
    static_for<2>([&](auto s) {
      const int kc = 32 * s.value + lg8;
      static_for<TPW>([&](auto t) {
        const bf16x8 eh = lds8(&Eh[16 * t.value + lr][kc]);
        const bf16x8 el = lds8(&El[16 * t.value + lr][kc]);
        static_for<2>([&](auto j) {
          sacc[t.value][j.value] = mfma16(kt[j.value][s.value], eh, sacc[t.value][j.value]);
          sacc[t.value][j.value] = mfma16(kt[j.value][s.value], el, sacc[t.value][j.value]);
        });
      });
    });
    load_kt(cn);
    write_state();  // every wave read S0 before the R^T barrier

    // ---- Y^T = gamma X_Q^T + U^T P^T (rows x this wave's 16 tokens)
    f32x4 y0[TPW], y1[TPW];
#pragma unroll
    for (int t = 0; t < TPW; ++t) y0[t] = y1[t] = z;
    static_for<2>([&](auto s) {
      if (s.value == 1 && !full_rows) return;
      const int kc = 32 * s.value + lg8;
      static_for<TPW>([&](auto t) {
        const bf16x8 uh = lds8(&Uh[16 * t.value + lr][kc]);
        y0[t.value] = mfma16(uh, o.ph[s.value], y0[t.value]);
        y1[t.value] = mfma16(lds8(&Ul[16 * t.value + lr][kc]), o.ph[s.value], y1[t.value]);
        y1[t.value] = mfma16(uh, o.pl[s.value], y1[t.value]);
      });
    });
    load_p(cn);
    static_for<TPW>([&](auto t) {
      const f32x4 yv = gy * (xq0[t.value] + xq1[t.value]) + (y0[t.value] + y1[t.value]);
      const bf16x4 yb = __builtin_convertvector(yv, bf16x4);
      __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u32x2, yb), y_cur, off_y + 32 * t.value, 0, 0);
    });
    y_cur = cn.y;
    store_gates();  // the next chunk's
  }

#pragma unroll
  for (int t = 0; t < TPW; ++t)
#pragma unroll
    for (int j = 0; j < 2; ++j)
      *reinterpret_cast<f32x4*>(p.state_out + (srow + 16 * t) * DK + 32 * wave + 16 * j + 4 * lq) = sacc[t][j];
}

// Bytes of the records (every chunk slot of a packed call, which bounds the
// unpacked count too); the sequence order follows them.
size_t record_bytes(int64_t n_seqs, int64_t n_tok, int64_t Hv);

bool ordered(int64_t n_seqs) { return n_seqs > 1 && n_seqs <= kOrderMax; }

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
  const size_t order = ordered(n_seqs) ? (static_cast<size_t>(n_seqs) * 4 + 255) / 256 * 256 : 0;
  return record_bytes(n_seqs, n_tok, Hv) + order;
}

// The fused conv prologue's workspace: gdn_chunk_fwd's, then the v rows the
// prep writes for the scan ([n_tok][Hv][Dv] bf16).
extern "C" size_t gdn_chunk_conv_workspace_bytes(int64_t n_seqs, int64_t n_tok, int64_t Hv, int64_t Dk,
                                                 int64_t Dv, int64_t chunk) {
  const size_t base = gdn_chunk_workspace_bytes(n_seqs, n_tok, Hv, Dk, Dv, chunk);
  if (base == 0 && !(n_seqs == 0 && chunk == CH && Dk == DK && Dv == DV && n_tok >= 0 && Hv > 0)) return 0;
  return base + (static_cast<size_t>(n_tok) * Hv * DV * 2 + 255) / 256 * 256;
}

// ------------------------------------------------ no-allocation entry point
//
// gdn_chunk_fwd with the chunk records in a file-scope device array instead
// of a caller's workspace, for callers that cannot allocate device memory
// (code under HIP graph capture, serving loops that forbid allocation).  The
// array is kScratchBytes; every GPU the library runs on holds its own copy
// (at its own address) until the process ends.  Its address is taken once
// per device, on the entry point's first call there with that device
// current, by hipGetSymbolAddress; the name `scratch` itself is a host-side
// stand-in and is never passed to a kernel.  The records need no clearing:
// the prep writes every record entry the scan reads.  All calls on one GPU
// share the array, so calls that overlap on one GPU (different streams, or
// an unfinished call's scan) race on it.

constexpr size_t kScratchBytes = size_t(64) << 20;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

}  // namespace

static int scratch_on_current_device(void** out) {
  using gdn_host::fail;
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail(GDN_ERR_LAUNCH, "gdn_chunk_fwd_noalloc: hipGetDevice: %s", hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices)
    return fail(GDN_ERR_UNSUPPORTED, "gdn_chunk_fwd_noalloc: device %d above %d", dev, kMaxDevices - 1);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || ptr == nullptr)
      return fail(GDN_ERR_LAUNCH, "gdn_chunk_fwd_noalloc: hipGetSymbolAddress(scratch) on device %d: %s", dev,
                  hipGetErrorString(e));
    if (!gdn_host::aligned(ptr, 256))
      return fail(GDN_ERR_LAUNCH, "gdn_chunk_fwd_noalloc: scratch on device %d is not 256-byte aligned", dev);
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  return GDN_OK;
}


namespace {

size_t record_bytes(int64_t n_seqs, int64_t n_tok, int64_t Hv) {
  return static_cast<size_t>(max_chunks(n_seqs, n_tok, true)) * static_cast<size_t>(Hv) * kRecBytes;
}

constexpr unsigned kPhasePrep = 1, kPhaseScan = 2;

// The conv prologue's arguments, for the prep that fuses it (as in
// gdn_conv_prologue: qkv rows of C = 2 Hk Dk + Hv Dv bf16 channels,
// qkv_stride elements apart; taps [C][4]; conv states [n_seqs][3][C] bf16).
struct ConvArgs {
  const void* qkv;
  int64_t qkv_stride;
  const void* w;
  int w_dtype;
  const void* cs_in;
  void* cs_out;
  float eps;
};

// Validates the arguments and enqueues the phases selected by `phases`
// (the same checks for every phase, so a prep and a scan issued separately
// with the same arguments see the same records).  With `use_scratch` the
// records go to the library's static scratch array on the current device
// instead of `workspace` (checked against its size before any HIP call).
int chunk_fwd(const void* q, const void* k, const void* v, int qkv_dtype, int gate_mode, const void* gx,
              const void* gy, int gate_dtype, int64_t gate_stride, const void* A_log, const void* dt_bias,
              int param_dtype, const uint8_t* mask, const float* state_in, void* y, float* state_out, const int32_t* state_index,
              int64_t n_slots, const int32_t* cu_seqlens, int64_t n_seqs, int64_t n_tok, int64_t Hk, int64_t Hv,
              int64_t Dk, int64_t Dv, int64_t chunk, void* workspace, size_t workspace_bytes, void* stream,
              unsigned phases, bool use_scratch = false, const ConvArgs* conv = nullptr) {
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
  const bool packed = cu_seqlens != nullptr;
  if (!packed && n_seqs > 0 && n_tok % n_seqs != 0)
    return fail(GDN_ERR_INVALID, "gdn_chunk_fwd: n_tok=%lld is not n_seqs=%lld rows of equal length",
                (long long)n_tok, (long long)n_seqs);
  if (n_tok > 0 && ((conv == nullptr && (!q || !k || !v)) || !gx || !gy || !y))
    return fail(GDN_ERR_INVALID, "gdn_chunk_fwd: q, k, v, gates and y are required");
  const int64_t C = 2 * Hk * DK + Hv * DV;
  if (conv != nullptr) {
    if ((n_tok > 0 && !conv->qkv) || !conv->w)
      return fail(GDN_ERR_INVALID, "gdn_chunk_fwd_conv: qkv and the conv weight are required");
    if (conv->w_dtype != GDN_DTYPE_BF16 && conv->w_dtype != GDN_DTYPE_F32)
      return fail(GDN_ERR_UNSUPPORTED, "gdn_chunk_fwd_conv: the conv weight must be bf16 or fp32");
    if (conv->qkv_stride != 0 && (conv->qkv_stride < C || conv->qkv_stride % 8 != 0))
      return fail(GDN_ERR_INVALID, "gdn_chunk_fwd_conv: qkv_stride=%lld must be >= C=%lld and a multiple of 8",
                  (long long)conv->qkv_stride, (long long)C);
    if (conv->cs_out != nullptr && conv->cs_out == conv->cs_in)
      return fail(GDN_ERR_INVALID, "gdn_chunk_fwd_conv: conv_state_out must not alias conv_state_in");
    if (!(conv->eps >= 0.0f)) return fail(GDN_ERR_INVALID, "gdn_chunk_fwd_conv: eps must be >= 0");
    if (!gdn_host::aligned(conv->qkv, 16) || !gdn_host::aligned(conv->w, 16) ||
        !gdn_host::aligned(conv->cs_in, 16) || !gdn_host::aligned(conv->cs_out, 16))
      return fail(GDN_ERR_INVALID, "gdn_chunk_fwd_conv: misaligned pointer");
  }
  if (!state_out) return fail(GDN_ERR_INVALID, "gdn_chunk_fwd: state_out is required");
  if (gate_stride != 0 && gate_stride < Hv)
    return fail(GDN_ERR_INVALID, "gdn_chunk_fwd: gate_stride=%lld is below Hv=%lld", (long long)gate_stride,
                (long long)Hv);
  if (state_index != nullptr && (n_slots < 0 || n_slots > INT32_MAX))
    return fail(GDN_ERR_INVALID, "gdn_chunk_fwd: n_slots=%lld out of range", (long long)n_slots);
  if (n_seqs == 0) return GDN_OK;
  const size_t need = conv != nullptr ? gdn_chunk_conv_workspace_bytes(n_seqs, n_tok, Hv, Dk, Dv, chunk)
                                      : gdn_chunk_workspace_bytes(n_seqs, n_tok, Hv, Dk, Dv, chunk);
  if (use_scratch) {
    if (need > kScratchBytes)
      return fail(GDN_ERR_UNSUPPORTED,
                  "gdn_chunk_fwd_noalloc: %zu bytes of chunk records exceed the static scratch of %zu bytes "
                  "(n_seqs=%lld, n_tok=%lld, Hv=%lld); use gdn_chunk_fwd with a workspace",
                  need, kScratchBytes, (long long)n_seqs, (long long)n_tok, (long long)Hv);
  } else if (workspace == nullptr || workspace_bytes < need) {
    return fail(GDN_ERR_INVALID, "gdn_chunk_fwd: workspace of %zu bytes is below the %zu needed", workspace_bytes,
                need);
  }
  if ((!use_scratch && !gdn_host::aligned(workspace, 256)) ||
      (conv == nullptr && (!gdn_host::aligned(q, 16) || !gdn_host::aligned(k, 16) || !gdn_host::aligned(v, 16))) ||
      !gdn_host::aligned(state_in, 16) || !gdn_host::aligned(state_out, 16))
    return fail(GDN_ERR_INVALID, "gdn_chunk_fwd: misaligned pointer");
  if (n_tok > INT32_MAX / 2 || n_seqs > 65535 || Hv > 65535 || max_chunks(n_seqs, n_tok, packed) * Hv >= INT32_MAX ||
      (DV / DVT) * (Hv * n_seqs + 8 * (Hv / Hk)) > INT32_MAX)
    return fail(GDN_ERR_UNSUPPORTED, "gdn_chunk_fwd: problem too large");
  if (use_scratch) {
    const int rc = scratch_on_current_device(&workspace);
    if (rc != GDN_OK) return rc;
  }

  ChunkParams p;
  p.q = static_cast<const uint16_t*>(q);
  p.k = static_cast<const uint16_t*>(k);
  p.v = static_cast<const uint16_t*>(v);
  p.ga.gx = gx;
  p.ga.gy = gy;
  p.ga.ld = gate_stride > 0 ? gate_stride : Hv;
  p.ga.A_log = A_log;
  p.ga.dt_bias = dt_bias;
  p.ga.mode = gate_mode;
  p.ga.gdt = gate_dtype;
  p.ga.pdt = param_dtype;
  p.state_in = state_in;
  p.y = static_cast<uint16_t*>(y);
  p.state_out = state_out;
  p.state_index = state_index;
  p.n_slots = state_index != nullptr ? static_cast<int>(n_slots) : 0;
  p.cu = cu_seqlens;
  p.n_seqs = static_cast<int>(n_seqs);
  p.n_tok = static_cast<int>(n_tok);
  p.T = packed ? 0 : static_cast<int>(n_tok / n_seqs);
  p.Hk = static_cast<int>(Hk);
  p.Hv = static_cast<int>(Hv);
  p.group = static_cast<int>(Hv / Hk);
  p.ws = static_cast<unsigned char*>(workspace);
  p.order = packed && ordered(n_seqs) ? reinterpret_cast<int32_t*>(p.ws + record_bytes(n_seqs, n_tok, Hv)) : nullptr;
  p.mask = mask;
  p.qkv = nullptr;
  p.conv_w = nullptr;
  p.cs_in = nullptr;
  p.cs_out = nullptr;
  p.v_out = nullptr;
  p.qkv_ld = 0;
  p.C = static_cast<int>(C);
  p.conv_eps = 0.0f;
  if (conv != nullptr) {
    // v rows after the records and the order table; the scan reads them as p.v
    p.v_out = reinterpret_cast<uint16_t*>(p.ws + gdn_chunk_workspace_bytes(n_seqs, n_tok, Hv, Dk, Dv, chunk));
    p.v = p.v_out;
    p.q = p.k = nullptr;
    p.qkv = static_cast<const uint16_t*>(conv->qkv);
    p.qkv_ld = conv->qkv_stride > 0 ? conv->qkv_stride : C;
    p.conv_w = conv->w;
    p.cs_in = static_cast<const uint16_t*>(conv->cs_in);
    p.cs_out = static_cast<uint16_t*>(conv->cs_out);
    p.conv_eps = conv->eps;
  }

  hipStream_t st = static_cast<hipStream_t>(stream);
  const int64_t chunks = max_chunks(n_seqs, n_tok, packed);
  if (conv != nullptr && chunks == 0 && (phases & kPhasePrep)) {
    // rows of no tokens: the prologue alone passes the conv states through
    // (it writes no q, k or v; the workspace stands in for them)
    const void* qkv = conv->qkv != nullptr ? conv->qkv : workspace;  // not read without tokens
    const int rc = gdn_conv_prologue(qkv, GDN_DTYPE_BF16, conv->qkv_stride, conv->cs_in, conv->w,
                                     conv->w_dtype, nullptr, nullptr, workspace, workspace, workspace, conv->cs_out,
                                     n_seqs, 0, Hk, Hv, Dk, Dv, KTAP, conv->eps, stream);
    if (rc != GDN_OK) return rc;
  }
  // More scan workgroups than CUs (several per CU): K^T from LDS (fewer
  // operand bytes per CU); else the record's K^T (a shorter chain per chunk).
  const bool kt_lds = static_cast<int64_t>(kTiles) * n_seqs * Hv > kCUs;
  if ((phases & kPhasePrep) && chunks > 0) {
    // one workgroup per (chunk slot, v-head), and one more that orders packed sequences
    const dim3 grid(static_cast<unsigned>(chunks * Hv + (p.order != nullptr ? 1 : 0)));
    // (the fused prologue takes no mask: conv != null implies mask == null)
    const int cv = conv == nullptr ? 0 : (conv->w_dtype == GDN_DTYPE_F32 ? 2 : 1);
    const bool masked = mask != nullptr;
    if (kt_lds) {
      if (masked) hipLaunchKernelGGL((chunk_prep_kernel<true, 0, true>), grid, dim3(256), 0, st, p);
      else if (cv == 0) hipLaunchKernelGGL((chunk_prep_kernel<true, 0, false>), grid, dim3(256), 0, st, p);
      else if (cv == 1) hipLaunchKernelGGL((chunk_prep_kernel<true, 1, false>), grid, dim3(256), 0, st, p);
      else hipLaunchKernelGGL((chunk_prep_kernel<true, 2, false>), grid, dim3(256), 0, st, p);
    } else {
      if (masked) hipLaunchKernelGGL((chunk_prep_kernel<false, 0, true>), grid, dim3(256), 0, st, p);
      else if (cv == 0) hipLaunchKernelGGL((chunk_prep_kernel<false, 0, false>), grid, dim3(256), 0, st, p);
      else if (cv == 1) hipLaunchKernelGGL((chunk_prep_kernel<false, 1, false>), grid, dim3(256), 0, st, p);
      else hipLaunchKernelGGL((chunk_prep_kernel<false, 2, false>), grid, dim3(256), 0, st, p);
    }
    const int rc = gdn_host::check_launch("gdn_chunk_fwd/prep");
    if (rc != GDN_OK) return rc;
  }
  // whole GQA units per XCD (a unit never spans two sequences: Hv % group == 0)
  const int64_t heads = n_seqs * Hv, unit = Hv / Hk;
  // Two tiles per workgroup when the tiles outnumber the CUs and every
  // sequence has the same length.  Packed sequences keep one: their longest
  // chain bounds the scan, and a two-tile workgroup's chunk takes about 1.8x
  // as long (measured at T=4096: B=2 153 against 167 us, B=4 260 against
  // 333 us, but the 1024/2560/7168 packed step 361 against 356 us).
  const int tpw = kt_lds && !packed ? 2 : 1;
  const int64_t scan_blocks = (kTiles / tpw) * kXcds * unit * ((heads + kXcds * unit - 1) / (kXcds * unit));
  if (!(phases & kPhaseScan)) return GDN_OK;
  const dim3 sgrid(static_cast<unsigned>(scan_blocks));
  if (mask != nullptr) {
    if (tpw == 2) hipLaunchKernelGGL((chunk_scan_kernel<true, 2, true>), sgrid, dim3(256), 0, st, p);
    else if (kt_lds) hipLaunchKernelGGL((chunk_scan_kernel<true, 1, true>), sgrid, dim3(256), 0, st, p);
    else hipLaunchKernelGGL((chunk_scan_kernel<false, 1, true>), sgrid, dim3(256), 0, st, p);
  } else {
    if (tpw == 2) hipLaunchKernelGGL((chunk_scan_kernel<true, 2, false>), sgrid, dim3(256), 0, st, p);
    else if (kt_lds) hipLaunchKernelGGL((chunk_scan_kernel<true, 1, false>), sgrid, dim3(256), 0, st, p);
    else hipLaunchKernelGGL((chunk_scan_kernel<false, 1, false>), sgrid, dim3(256), 0, st, p);
  }
  return gdn_host::check_launch("gdn_chunk_fwd/scan");
}

}  // namespace

#define GDN_CHUNK_PARAMS                                                                                        \
  const void *q, const void *k, const void *v, int qkv_dtype, int gate_mode, const void *gx, const void *gy,   \
      int gate_dtype, int64_t gate_stride, const void *A_log, const void *dt_bias, int param_dtype,             \
      const uint8_t *mask, const float *state_in, void *y, float *state_out, const int32_t *state_index, int64_t n_slots,            \
      const int32_t *cu_seqlens, int64_t n_seqs, int64_t n_tok, int64_t Hk, int64_t Hv, int64_t Dk, int64_t Dv, \
      int64_t chunk, void *workspace, size_t workspace_bytes, void *stream
#define GDN_CHUNK_ARGS                                                                                        \
  q, k, v, qkv_dtype, gate_mode, gx, gy, gate_dtype, gate_stride, A_log, dt_bias, param_dtype, mask, state_in, y, \
      state_out, state_index, n_slots, cu_seqlens, n_seqs, n_tok, Hk, Hv, Dk, Dv, chunk, workspace,           \
      workspace_bytes, stream

extern "C" int gdn_chunk_fwd(GDN_CHUNK_PARAMS) { return chunk_fwd(GDN_CHUNK_ARGS, kPhasePrep | kPhaseScan); }

extern "C" int gdn_chunk_prep(GDN_CHUNK_PARAMS) { return chunk_fwd(GDN_CHUNK_ARGS, kPhasePrep); }

extern "C" int gdn_chunk_scan(GDN_CHUNK_PARAMS) { return chunk_fwd(GDN_CHUNK_ARGS, kPhaseScan); }

extern "C" int gdn_chunk_fwd_conv(const void* qkv, int64_t qkv_stride, const void* conv_w, int conv_w_dtype,
                                  const void* conv_state_in, void* conv_state_out, float eps, int gate_mode,
                                  const void* gx, const void* gy, int gate_dtype, int64_t gate_stride,
                                  const void* A_log, const void* dt_bias, int param_dtype, const float* state_in,
                                  void* y, float* state_out, const int32_t* state_index, int64_t n_slots,
                                  const int32_t* cu_seqlens, int64_t n_seqs, int64_t n_tok, int64_t Hk, int64_t Hv,
                                  int64_t Dk, int64_t Dv, int64_t chunk, void* workspace, size_t workspace_bytes,
                                  void* stream) {
  const ConvArgs conv{qkv, qkv_stride, conv_w, conv_w_dtype, conv_state_in, conv_state_out, eps};
  return chunk_fwd(nullptr, nullptr, nullptr, GDN_DTYPE_BF16, gate_mode, gx, gy, gate_dtype, gate_stride, A_log,
                   dt_bias, param_dtype, nullptr, state_in, y, state_out, state_index, n_slots, cu_seqlens, n_seqs, n_tok, Hk,
                   Hv, Dk, Dv, chunk, workspace, workspace_bytes, stream, kPhasePrep | kPhaseScan, false, &conv);
}

extern "C" int gdn_chunk_fwd_noalloc(const void* q, const void* k, const void* v, int qkv_dtype, int gate_mode,
                                     const void* gx, const void* gy, int gate_dtype, int64_t gate_stride,
                                     const void* A_log, const void* dt_bias, int param_dtype, const uint8_t* mask,
                                     const float* state_in,
                                     void* y, float* state_out, const int32_t* state_index, int64_t n_slots,
                                     const int32_t* cu_seqlens, int64_t n_seqs, int64_t n_tok, int64_t Hk,
                                     int64_t Hv, int64_t Dk, int64_t Dv, int64_t chunk, void* stream) {
  return chunk_fwd(q, k, v, qkv_dtype, gate_mode, gx, gy, gate_dtype, gate_stride, A_log, dt_bias, param_dtype, mask,
                   state_in, y, state_out, state_index, n_slots, cu_seqlens, n_seqs, n_tok, Hk, Hv, Dk, Dv, chunk,
                   nullptr, 0, stream, kPhasePrep | kPhaseScan, true);
}
