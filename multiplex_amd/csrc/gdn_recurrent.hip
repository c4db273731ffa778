// Recurrent gated delta rule for decode, MTP verify and commit (gfx950).
//
// One launch advances independent (row, v-head) states by up to T tokens.
// The state S[Dv][Dk] of a (row, v-head) is fp32 and lives in VGPRs for the
// whole launch: it is read from HBM once and written at most once (plus the
// optional per-token snapshots).  Rows of S (one dv index each) are
// independent in the recurrence, so the kernel parallelises over dv:
//
//   * LPR lanes own one state row of Dk floats; lane `sub` holds the float4s
//     at offsets i*4*LPR + sub*4 (i < Dk/(4*LPR)).  The decode kernel uses
//     LPR = Dk/4 (one float4 per lane, 1 KB of contiguous state per load
//     instruction); the multi-token kernels use LPR = 8 (8 rows x 128
//     contiguous bytes per instruction, 32 rows per 4-wave workgroup, so a
//     token tile in LDS serves 32 rows).
//   * the two dot products per token (S k and S q) are summed over the row's
//     lanes in one order for both layouts (row_dot): a state steps
//     bit-identically in the decode and the multi-token kernels.
//   * the grid is (dv blocks, Hv, rows).
//
// Every load is branch-free (clamped addresses; a device-resident zero row
// for a missing state, a constant 1 for a missing mask), and the state load
// is issued first with a token's inputs right behind it, none of them used
// before all are issued, so one memory latency covers both.  Algorithmic traffic per (row, head): Dv*Dk*4 bytes read + the same
// written (once), plus q/k/v/y/gates per token; the kernel is HBM-bound.
#include "gdn_common.hpp"

namespace {

using namespace gdn;

constexpr int kLanesPerRow = 8;
constexpr int kMaxDk = 256;

// Read-only stand-ins for absent operands (loads stay unconditional).
__device__ const float kZeroRow[kMaxDk] = {};
__device__ const uint8_t kActive = 1;

// Global-memory views of a pointer that may be either a kernel argument or
// one of the stand-ins above: a select between the two is a generic pointer,
// whose loads would be flat loads, and a flat load also counts on the
// scalar-load counter, so the gate parameters' scalar loads would wait for it.
typedef __attribute__((address_space(1))) const f32x4 gbl_f32x4;
typedef __attribute__((address_space(1))) const uint8_t gbl_u8;
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

struct RecParams {
  // the fields the decode kernel reads come first (two 64-byte parameter loads)
  const void* q;
  const void* k;
  const void* v;
  const float* state_in;
  float* state_out;
  void* y;
  GateArgs ga;
  int Hk, Hv, Dv, group;     // group = Hv / Hk
  unsigned group_magic;      // ceil(2^31 / group): hv / group = (hv * magic) >> 31
  int wg_rows;               // state rows per workgroup (decode kernel)
  int T, n_slots;
  const int32_t* state_index;  // slot of each row in pooled states, or NULL
  float* snapshots;
  const uint8_t* mask;
  const int32_t* cu_seqlens;
  const int32_t* commit_len;
  int y_from;  // tokens before it produce no y (tile kernel)
};

// A state row of Dk floats is spread over LPR lanes: lane `sub` holds the
// float4s at offsets i*4*LPR + sub*4, so one load instruction covers
// 64/LPR rows x 16*LPR contiguous bytes.
template <int EPL, int LPR = kLanesPerRow>
__device__ __forceinline__ void store_row(float* dst, int sub, const float (&s)[EPL]) {
  constexpr int NV = EPL / 4;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    f32x4 x = {s[4 * i], s[4 * i + 1], s[4 * i + 2], s[4 * i + 3]};
    __builtin_nontemporal_store(x, reinterpret_cast<f32x4*>(dst + i * 4 * LPR + sub * 4));
  }
}

// Shared preamble of the multi-token kernels: row / head / sequence
// bookkeeping (8 lanes per state row).
struct RowCtx {
  int sub, dv, dv_c, hv, hk, row, L, commit, steps;
  bool row_ok, write_state, want_y;
  bool skip;  // pooled row with a slot outside the pool: not processed
  int64_t tok0, srow, srow_c;
};

template <int DK>
__device__ __forceinline__ RowCtx row_ctx(const RecParams& p) {
  RowCtx c;
  c.sub = threadIdx.x & (kLanesPerRow - 1);
  c.dv = blockIdx.x * (blockDim.x / kLanesPerRow) + threadIdx.x / kLanesPerRow;
  c.row_ok = c.dv < p.Dv;
  c.dv_c = c.row_ok ? c.dv : p.Dv - 1;  // loads use a valid row; stores check row_ok
  c.hv = blockIdx.y;
  c.row = blockIdx.z;
  c.hk = c.hv / p.group;
  if (p.cu_seqlens != nullptr) {
    // Offsets from a device tensor are not validated on the host: each
    // sequence is clamped into [0, T] (T = the packed token count), so a bad
    // table gives wrong rows but never an access outside the buffers.
    const int start = min(max(p.cu_seqlens[c.row], 0), p.T);
    const int end = min(max(p.cu_seqlens[c.row + 1], start), p.T);
    c.tok0 = start;
    c.L = end - start;
  } else {
    c.tok0 = static_cast<int64_t>(c.row) * p.T;
    c.L = p.T;
  }
  c.write_state = p.state_out != nullptr;
  c.commit = c.L;
  if (p.commit_len != nullptr) {
    // A negative length skips the row: in place (state_out == state_in) it
    // is not written at all; into a separate state_out it is copied
    // unchanged (commit 0), so no output row is left unwritten.
    const int cl = p.commit_len[c.row];
    if (cl < 0 && p.state_out == p.state_in) c.write_state = false;
    c.commit = cl < 0 ? 0 : (cl < c.L ? cl : c.L);
  }
  c.want_y = p.y != nullptr;
  const bool need_all = c.want_y || (p.snapshots != nullptr);
  c.steps = need_all ? c.L : (c.write_state ? c.commit : 0);
  int slot = c.row;
  c.skip = false;
  if (p.state_index != nullptr) {
    slot = p.state_index[c.row];
    c.skip = slot < 0 || slot >= p.n_slots;
  }
  c.srow = ((static_cast<int64_t>(slot) * p.Hv + c.hv) * p.Dv + c.dv) * DK;
  c.srow_c = ((static_cast<int64_t>(slot) * p.Hv + c.hv) * p.Dv + c.dv_c) * DK;
  return c;
}

template <int DK>
__device__ __forceinline__ void load_state(const RecParams& p, const RowCtx& c, float (&s)[DK / kLanesPerRow]) {
  constexpr int NV = DK / kLanesPerRow / 4;
  const float* src = p.state_in != nullptr ? p.state_in + c.srow_c : kZeroRow;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const f32x4 x = __builtin_nontemporal_load((gbl_f32x4*)(src + i * 4 * kLanesPerRow + c.sub * 4));
    s[4 * i] = x.x;
    s[4 * i + 1] = x.y;
    s[4 * i + 2] = x.z;
    s[4 * i + 3] = x.w;
  }
}

// row_ror:8 inside a 16-lane row: lane l reads lane l ^ 8.
#define GDN_DPP_ROW_ROR8 0x128

// Dot product of a lane's slice of a state row with the matching slice of x,
// summed over the row's LPR lanes in one fixed order for both lane layouts,
// so that the decode kernel (LPR = Dk/4) and the multi-token kernels
// (LPR = 8) step a state bit-identically.  The order: the row's Dk columns
// form Dk/32 blocks of 32; inside a block, the 4 columns of each group g
// (g = (column/4) % 8) are a 4-term fma chain; the blocks' chains of one
// group are added in a balanced pairwise tree (blocks 2m and 2m+1 first);
// the 8 group sums are then added by sum8.  With LPR = 8 a lane holds all
// blocks of its group and the tree is in-lane; with LPR = Dk/4 lane
// 8*block + g holds one chain, and blocks 2m, 2m+1 are 8 lanes apart (DPP
// row_ror:8), pairs of those 16 lanes apart (permlane16 swap), quads 32
// lanes apart (permlane32 swap).
template <int EPL, int LPR>
__device__ __forceinline__ float row_dot(const float (&s)[EPL], const float (&x)[EPL]) {
  constexpr int NV = EPL / 4;
  static_assert(LPR == 8 || NV == 1, "a row spans 8 lanes or holds one float4 per lane");
  float part[NV];
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    float c = 0.0f;
#pragma unroll
    for (int j = 0; j < 4; ++j) c = fmaf(s[4 * i + j], x[4 * i + j], c);
    part[i] = c;
  }
#pragma unroll
  for (int w = 1; w < NV; w *= 2) {
#pragma unroll
    for (int i = 0; i + w < NV; i += 2 * w) part[i] += part[i + w];
  }
  float r = part[0];
  if constexpr (LPR >= 16) r += dpp_f<GDN_DPP_ROW_ROR8>(r);
  if constexpr (LPR >= 32) {
    const auto h = __builtin_amdgcn_permlane16_swap(__float_as_uint(r), __float_as_uint(r), false, false);
    r = __uint_as_float(h[0]) + __uint_as_float(h[1]);
  }
  if constexpr (LPR >= 64) {
    const auto h = __builtin_amdgcn_permlane32_swap(__float_as_uint(r), __float_as_uint(r), false, false);
    r = __uint_as_float(h[0]) + __uint_as_float(h[1]);
  }
  return sum8(r);
}

// One token of the recurrence on a lane's slice of a state row:
// S <- g S;  kv = S k;  S <- S + beta (v - kv) k^T  (kv by row_dot).
template <int EPL, int LPR = kLanesPerRow>
__device__ __forceinline__ void step_row(float (&s)[EPL], const float (&k)[EPL], float v, float g,
                                          float beta) {
#pragma unroll
  for (int e = 0; e < EPL; ++e) s[e] *= g;
  const float kv = row_dot<EPL, LPR>(s, k);
  const float delta = beta * (v - kv);
#pragma unroll
  for (int e = 0; e < EPL; ++e) s[e] = fmaf(k[e], delta, s[e]);
}

// Decode body (T <= 1 token per row, rows not packed): no LDS, no barriers,
// no loop.  A state row is spread over Dk/4 lanes, one float4 each, so a
// load instruction of a wave covers 1 KB of contiguous state (at Dk = 128:
// two rows) and a wave streams exactly one such unit: that shape streams the
// in-place read + write of a 128 MiB state at ~6.7-6.9 TB/s, against ~6.2
// TB/s for waves that hold two or more units (8 lanes per row with four
// float4 each, or one float4 per lane over several row pairs).  With that
// many short waves the per-wave scalar work is what limits, so the body is
// straight-line, indexes in 32 bits (the host bounds every tensor below 2^31
// elements), divides hv by the group with a multiplier, and takes the rows
// per workgroup from the parameters.  The state load is issued first and
// the token's loads right behind it, so one latency covers both.  Dot
// products over a row are row_dot, in the order of the multi-token kernels.
//
// MODE: kDecodeAny takes every option at run time.  kDecodeLean and
// kDecodeLeanPooled are the serving step with every option fixed -- T = 1,
// state_in and state_out given, y wanted, no mask, commit lengths or
// snapshots, raw gates of a typed format (with 16-bit gates and v: 4-byte
// aligned, even gate stride, Hv and Dv) -- without (with) a pool-slot table:
// the same arithmetic with those checks removed, so the same results.
enum DecodeMode { kDecodeAny = 0, kDecodeLean = 1, kDecodeLeanPooled = 2 };

template <int DK, int DT, int GF, int MODE>
__global__ __launch_bounds__(256) void recurrent_kernel(const RecParams p) {
  constexpr int LPR = DK / 4;  // lanes per state row, one float4 each
  constexpr bool lean = MODE != kDecodeAny;
  static_assert(!lean || GF != GF_ANY, "the lean decode takes raw gates of a typed format");
  float s[4];
  const int sub = threadIdx.x & (LPR - 1);
  const int row = blockIdx.z, hv = blockIdx.y;
  const int hk = static_cast<int>((static_cast<uint64_t>(hv) * p.group_magic) >> 31);
  const int dv = blockIdx.x * p.wg_rows + static_cast<int>(threadIdx.x) / LPR;
  const bool row_ok = dv < p.Dv;
  const int dv_c = row_ok ? dv : p.Dv - 1;  // loads use a valid row; stores check row_ok
  int slot = row;
  if (MODE == kDecodeLeanPooled || (MODE == kDecodeAny && p.state_index != nullptr)) {
    slot = p.state_index[row];
    if (slot < 0 || slot >= p.n_slots) return;  // uniform: not processed
  }
  const unsigned srow_c = (static_cast<unsigned>(slot) * p.Hv + hv) * p.Dv + dv_c;
  {
    const float* src = lean || p.state_in != nullptr ? p.state_in + static_cast<size_t>(srow_c) * DK : kZeroRow;
    const f32x4 x = __builtin_nontemporal_load((gbl_f32x4*)(src + sub * 4));
    s[0] = x.x;
    s[1] = x.y;
    s[2] = x.z;
    s[3] = x.w;
  }
  float al, db;
  param_load_raw<GF, DT>(p.ga, hv, al, db);

  // T is 0 or 1 here: the token of row `row` is token `row`.  A negative
  // commit length skips the row: in place it is not written at all; into a
  // separate state_out it is copied unchanged (commit 0).
  const int L = lean ? 1 : p.T;
  bool write_state = lean || p.state_out != nullptr;
  int commit = L;
  if (!lean && p.commit_len != nullptr) {
    const int cl = p.commit_len[row];
    if (cl < 0 && p.state_out == p.state_in) write_state = false;
    commit = cl < 0 ? 0 : min(cl, L);
  }
  const bool want_y = lean || p.y != nullptr;
  const bool snaps = !lean && p.snapshots != nullptr;
  const bool step = lean || (L > 0 && (want_y || snaps || (write_state && commit > 0)));
  const unsigned srow = srow_c + (dv - dv_c);  // the row the stores address (row_ok)

  // With two state rows per wave (Dk = 128) both rows read the same k and q:
  // one load instruction brings k to the low half-wave and q to the high one
  // (kq_merged), and a permlane32 swap of each dword then hands every lane
  // both, when they are used.
  constexpr bool kq_merged = LPR == 32 && DT != GDN_DTYPE_F32;
  typename IO<DT>::raw4 kr = {}, qr = {};
  typename IO<DT>::raw1 vr = {};
  float gx = 0.0f, gy = 0.0f;
  uint8_t m = 0;
  if (step) {
    const unsigned kq = (static_cast<unsigned>(row) * p.Hk + hk) * DK + sub * 4;
    if constexpr (kq_merged) {
      kr = IO<DT>::load4_raw((threadIdx.x & 32) && want_y ? p.q : p.k, kq);
    } else {
      kr = IO<DT>::load4_raw(p.k, kq);
      qr = IO<DT>::load4_raw(want_y ? p.q : p.k, kq);  // k stands in when no output is wanted
    }
    const unsigned gi = static_cast<unsigned>(row) * static_cast<unsigned>(p.ga.ld) + hv;
    if constexpr (lean && DT != GDN_DTYPE_F32) {
      // The gates and the v of the wave's two rows are wave-uniform 16-bit
      // values: each is read with a scalar load of the aligned dword holding
      // it (the host takes this body only when the other half of each dword
      // is inside the same tensor: 4-byte aligned pointers, even gate stride,
      // Hv and Dv), which keeps three vector loads off every wave.
      static_assert(LPR == 32, "two state rows per wave");
      const int wave0 = static_cast<int>(blockIdx.x) * p.wg_rows +
                        2 * static_cast<int>(__builtin_amdgcn_readfirstlane(threadIdx.x >> 6));
      const int wdv = min(wave0, p.Dv - 2);
      const uint32_t vw =
          static_cast<const uint32_t*>(p.v)[((static_cast<unsigned>(row) * p.Hv + hv) * p.Dv + wdv) >> 1];
      const uint32_t aw = static_cast<const uint32_t*>(p.ga.gx)[gi >> 1];
      const uint32_t bw = static_cast<const uint32_t*>(p.ga.gy)[gi >> 1];
      vr = static_cast<uint16_t>((threadIdx.x & 32) ? vw >> 16 : vw);
      gx = IO<DT>::cvt1(static_cast<uint16_t>((gi & 1) ? aw >> 16 : aw));
      gy = IO<DT>::cvt1(static_cast<uint16_t>((gi & 1) ? bw >> 16 : bw));
    } else {
      vr = IO<DT>::load1_raw(p.v, (static_cast<unsigned>(row) * p.Hv + hv) * p.Dv + dv_c);
      gate_load<GF, DT>(p.ga, gi, gx, gy);
    }
    if (lean) {
      m = 1;
    } else {
      const uint8_t* mp = p.mask != nullptr ? p.mask + row : &kActive;
      m = *(gbl_u8*)mp;
    }
  }
  // the output pointer is read here, with the loads in flight, not at its
  // store (a parameter read there would be one more wait at the end of every
  // wave); the empty asm pins it, and comes after the loads above because
  // the compiler counts it as a possible memory write, after which no load
  // may become a scalar load
  void* yp = p.y;
  asm volatile("" : "+s"(yp));
  if (!lean && write_state && commit == 0 && row_ok)
    store_row<4, LPR>(p.state_out + static_cast<size_t>(srow) * DK, sub, s);
  if (!step) return;

  float yv = 0.0f;
  if (m != 0) {
    if constexpr (kq_merged) {
      // uniform here (step and m are per batch row), so every lane takes part
      const u32x2 w = __builtin_bit_cast(u32x2, kr);
      const auto lo = __builtin_amdgcn_permlane32_swap(w.x, w.x, false, false);
      const auto hi = __builtin_amdgcn_permlane32_swap(w.y, w.y, false, false);
      kr = __builtin_bit_cast(typename IO<DT>::raw4, u32x2{lo[0], hi[0]});
      qr = __builtin_bit_cast(typename IO<DT>::raw4, u32x2{lo[1], hi[1]});
    }
    const float ea = GF == GF_ANY && p.ga.mode == GDN_GATES_PRE ? 0.0f : exp_fast(al);
    float g, beta;
    gate_transform<GF>(p.ga.mode, gx, gy, ea, db, g, beta);
    const f32x4 k4 = IO<DT>::cvt4(kr);
    const float kf[4] = {k4.x, k4.y, k4.z, k4.w};
    step_row<4, LPR>(s, kf, IO<DT>::cvt1(vr), g, beta);
    if (want_y) {
      const f32x4 q4 = IO<DT>::cvt4(qr);
      const float qf[4] = {q4.x, q4.y, q4.z, q4.w};
      yv = row_dot<4, LPR>(s, qf);
    }
  }
  const unsigned yi = (static_cast<unsigned>(row) * p.Hv + hv) * p.Dv + dv;
  if (want_y && row_ok && sub == 0) IO<DT>::store1(yp, yi, yv);
  if (snaps && row_ok) store_row<4, LPR>(p.snapshots + static_cast<size_t>(yi) * DK, sub, s);
  if (write_state && commit == 1 && row_ok) store_row<4, LPR>(p.state_out + static_cast<size_t>(srow) * DK, sub, s);
}

// Multi-token body (verify, commit, packed rows): the workgroup (always 4
// waves, 32 state rows) stages a tile of TILE tokens -- k and q as fp32, the
// transformed gates, the mask and the v values of its rows -- in LDS, then
// every wave walks the tile from LDS.  The first tile's global loads are
// issued right behind the state stream, so both arrive within one latency.
// TILE is 4, 8 or 16, the smallest that holds the launch's tokens per row
// (16 for longer or packed rows): a larger tile than the tokens would re-read
// the last token into the unused slots.
constexpr int kTileMax = 16;
constexpr int kTileThreads = 256;
constexpr int kTileRows = kTileThreads / kLanesPerRow;  // 32

template <int DK, int DT, int GF, int TILE>
__global__ __launch_bounds__(kTileThreads) void recurrent_tile_kernel(const RecParams p) {
  constexpr int EPL = DK / kLanesPerRow;
  constexpr int NV = EPL / 4;
  constexpr int NK = TILE * DK / 4;                             // float4 of k (and q) in the tile
  constexpr int KV4 = (NK + kTileThreads - 1) / kTileThreads;   // ... per thread
  constexpr int NVV = TILE * kTileRows;                         // v values in the tile
  constexpr int VV = (NVV + kTileThreads - 1) / kTileThreads;   // ... per thread
  const RowCtx c = row_ctx<DK>(p);
  if (c.skip) return;  // uniform: a workgroup serves one row, before any barrier
  const int tid = threadIdx.x;
  const int dv0 = blockIdx.x * kTileRows;

  __shared__ __align__(16) float Kt[TILE][DK];
  __shared__ __align__(16) float Qt[TILE][DK];
  __shared__ float Vt[TILE][kTileRows];
  __shared__ float Gt[TILE], Bt[TILE];
  __shared__ uint8_t Mt[TILE];

  // The state load is issued first, then the parameters' and the first
  // tile's loads: loads complete in issue order, so the first use of a tile
  // value waits for one latency covering all of them.  Every load is
  // unconditional (q is read from k when no output is wanted): a load under
  // a branch sits in a block of its own, whose use the compiler would wait
  // for there, before the next load is issued.
  float s[EPL];
  load_state<DK>(p, c, s);
  float al, db;
  param_load_raw<GF, DT>(p.ga, c.hv, al, db);
  const void* qp = c.want_y ? p.q : p.k;

  typename IO<DT>::raw4 kr[KV4], qr[KV4];  // converted when written to LDS
  typename IO<DT>::raw1 vr[VV];
  float gx = 0.0f, gy = 0.0f;
  uint8_t mm = 1;
  float ea = 0.0f;
  // rows past the tile's n tokens re-read its last token (never used)
  auto issue_tile = [&](int t0, int n) {
#pragma unroll
    for (int it = 0; it < KV4; ++it) {
      const int i = min(tid + kTileThreads * it, NK - 1);
      const int j = i / (DK / 4), e = (i % (DK / 4)) * 4;
      const int64_t off = ((c.tok0 + t0 + min(j, n - 1)) * p.Hk + c.hk) * DK + e;
      kr[it] = IO<DT>::load4_raw(p.k, off);
      qr[it] = IO<DT>::load4_raw(qp, off);
    }
#pragma unroll
    for (int it = 0; it < VV; ++it) {
      const int i = min(tid + kTileThreads * it, NVV - 1);
      const int j = i / kTileRows, r = i % kTileRows;
      const int64_t tok = c.tok0 + t0 + min(j, n - 1);
      vr[it] = IO<DT>::load1_raw(p.v, (tok * p.Hv + c.hv) * p.Dv + min(dv0 + r, p.Dv - 1));
    }
    // threads tid < TILE keep token tid's gates and mask; the others load a
    // valid token too (no branch) and never use it
    {
      const int64_t tok = c.tok0 + t0 + min(tid, n - 1);
      gate_load<GF, DT>(p.ga, tok * p.ga.ld + c.hv, gx, gy);
      const uint8_t* mp = p.mask != nullptr ? p.mask + tok : &kActive;
      mm = *(gbl_u8*)mp;
    }
  };
  auto store_tile = [&]() {
#pragma unroll
    for (int it = 0; it < KV4; ++it) {
      const int i = tid + kTileThreads * it;
      if (i < NK) {
        const int j = i / (DK / 4), e = (i % (DK / 4)) * 4;
        *reinterpret_cast<f32x4*>(&Kt[j][e]) = IO<DT>::cvt4(kr[it]);
        if (c.want_y) *reinterpret_cast<f32x4*>(&Qt[j][e]) = IO<DT>::cvt4(qr[it]);
      }
    }
#pragma unroll
    for (int it = 0; it < VV; ++it) {
      const int i = tid + kTileThreads * it;
      if (i < NVV) Vt[i / kTileRows][i % kTileRows] = IO<DT>::cvt1(vr[it]);
    }
    if (tid < TILE) {
      float g, beta;
      gate_transform<GF>(p.ga.mode, gx, gy, ea, db, g, beta);
      Gt[tid] = g;
      Bt[tid] = beta;
      Mt[tid] = mm;
    }
  };

  if (c.steps > 0) issue_tile(0, min(TILE, c.steps));
  ea = GF == GF_ANY && p.ga.mode == GDN_GATES_PRE ? 0.0f : exp_fast(al);
  if (c.write_state && c.commit == 0 && c.row_ok) store_row<EPL>(p.state_out + c.srow, c.sub, s);

  const int rloc = threadIdx.x / kLanesPerRow;
  for (int t0 = 0; t0 < c.steps; t0 += TILE) {
    const int n = min(TILE, c.steps - t0);
    if (t0 > 0) {
      __syncthreads();  // the previous tile is consumed
      issue_tile(t0, n);
    }
    store_tile();
    __syncthreads();

    for (int j = 0; j < n; ++j) {
      const int t = t0 + j;
      const int64_t tok = c.tok0 + t;
      const bool y_here = c.want_y && t >= p.y_from;
      float yv = 0.0f;
      if (Mt[j] != 0) {
        float kf[EPL];
#pragma unroll
        for (int i = 0; i < NV; ++i) {
          const f32x4 x = *reinterpret_cast<const f32x4*>(&Kt[j][i * 32 + c.sub * 4]);
          kf[4 * i] = x.x;
          kf[4 * i + 1] = x.y;
          kf[4 * i + 2] = x.z;
          kf[4 * i + 3] = x.w;
        }
        step_row<EPL>(s, kf, Vt[j][rloc], Gt[j], Bt[j]);
        if (y_here) {
          float qf[EPL];
#pragma unroll
          for (int i = 0; i < NV; ++i) {
            const f32x4 x = *reinterpret_cast<const f32x4*>(&Qt[j][i * 32 + c.sub * 4]);
            qf[4 * i] = x.x;
            qf[4 * i + 1] = x.y;
            qf[4 * i + 2] = x.z;
            qf[4 * i + 3] = x.w;
          }
          yv = row_dot<EPL, kLanesPerRow>(s, qf);
        }
      }
      if (y_here && c.row_ok && c.sub == 0) IO<DT>::store1(p.y, (tok * p.Hv + c.hv) * p.Dv + c.dv, yv);
      if (p.snapshots != nullptr && c.row_ok) {
        store_row<EPL>(p.snapshots + ((tok * p.Hv + c.hv) * p.Dv + c.dv) * DK, c.sub, s);
      }
      if (c.write_state && t + 1 == c.commit && c.row_ok) store_row<EPL>(p.state_out + c.srow, c.sub, s);
    }
  }
}

// Speculative verify of T <= 8 draft tokens that writes no state.  With
// a_t = S0 k_t and b_t = S0 q_t per state row (2T dot products) and
// r(t,s) = g_{s+1} ... g_t (r(t,t) = 1), gamma_t = g_1 ... g_t, the
// recurrence unrolls to scalars per row:
//   delta_t = beta_t (v_t - gamma_t a_t - sum_{s<t} r(t,s) (k_s.k_t) delta_s)
//   y_t     = gamma_t b_t + sum_{s<=t} r(t,s) (k_s.q_t) delta_s
// so no intermediate state is formed: about half the VALU work of stepping
// the state through every token.  The per-head coefficients r(t,s) k_s.k_t
// and r(t,s) k_s.q_t come from products of g (no logarithms, so a decay that
// underflows to 0 stays exact) and are formed once per workgroup in LDS.  A
// masked token has g = 1, beta = 0 and y = 0.
constexpr int kVerifyMaxT = 8;

// Bit t set: token t of the row (t < T) is real and not masked, from a wave
// whose lane l holds the mask byte of token min(l, T - 1).  The verify
// kernels store a masked token's k, q and v as zeros: with g = 1 and
// beta = 0 alone, a non-finite value there would still reach the other
// tokens as 0 * inf in the coefficients, where the reference's where()
// keeps the masked step out entirely.
__device__ __forceinline__ uint32_t live_tokens(uint8_t lane_mask, int T) {
  const int lane = threadIdx.x & 63;
  return static_cast<uint32_t>(__builtin_amdgcn_ballot_w64(lane < T && lane_mask != 0));
}

// TM: tokens the kernel is built for (4 or kVerifyMaxT), T <= TM at run time.
template <int DK, int DT, int GF, int TM>
__global__ __launch_bounds__(kTileThreads) void verify_wy_kernel(const RecParams p) {
  constexpr int EPL = DK / kLanesPerRow;
  constexpr int NV = EPL / 4;
  static_assert(TM * kTileRows <= kTileThreads, "one v value per thread");
  const RowCtx c = row_ctx<DK>(p);
  if (c.skip) return;  // uniform: a workgroup serves one row, before any barrier
  const int tid = threadIdx.x;
  const int dv0 = blockIdx.x * kTileRows;
  const int T = c.L;  // 1 <= T <= TM on this path

  __shared__ __align__(16) float Ks[TM][DK];
  __shared__ __align__(16) float Qs[TM][DK];
  __shared__ float Vs[TM][kTileRows];
  __shared__ float Gs[TM], Bs[TM];          // g_t, beta_t (1 and 0 when masked)
  __shared__ float Gam[TM];                 // gamma_t
  __shared__ float Ckk[TM][TM], Ckq[TM][TM];
  __shared__ uint8_t Ms[TM];

  // The state row is issued first, then every token load (all
  // unconditional, with clamped addresses, kept as loaded bits until all are
  // issued): loads complete in issue order, so one latency covers them all.
  float s[EPL];
  load_state<DK>(p, c, s);
  float al, db;
  param_load_raw<GF, DT>(p.ga, c.hv, al, db);

  constexpr int NK4 = TM * DK / 4;  // float4 of k (and of q) in the tile
  constexpr int KV4 = (NK4 + kTileThreads - 1) / kTileThreads;
  typename IO<DT>::raw4 kr[KV4], qr[KV4];
  static_for<KV4>([&](auto it) {
    const int i = min(tid + kTileThreads * it.value, NK4 - 1);
    const int j = i / (DK / 4), e = (i % (DK / 4)) * 4;
    const int64_t off = ((c.tok0 + min(j, T - 1)) * p.Hk + c.hk) * DK + e;
    kr[it.value] = IO<DT>::load4_raw(p.k, off);
    qr[it.value] = IO<DT>::load4_raw(p.q, off);
  });
  typename IO<DT>::raw1 vr;
  float gx, gy;
  uint8_t mm;
  {
    const int j = min(tid / kTileRows, TM - 1), r = tid % kTileRows;
    const int64_t tok = c.tok0 + min(j, T - 1);
    vr = IO<DT>::load1_raw(p.v, (tok * p.Hv + c.hv) * p.Dv + min(dv0 + r, p.Dv - 1));
  }
  // threads tid < TM keep token tid's gates and mask; the others load a
  // valid token too and never use it
  {
    const int64_t tok = c.tok0 + min(tid, T - 1);
    gate_load<GF, DT>(p.ga, tok * p.ga.ld + c.hv, gx, gy);
    // the mask byte of token lane (the same token as tid in wave 0, the one
    // that uses mm), so that every wave can form the live-token bits
    const int64_t mtok = c.tok0 + min(static_cast<int>(tid & 63), T - 1);
    const uint8_t* mp = p.mask != nullptr ? p.mask + mtok : &kActive;
    mm = *(gbl_u8*)mp;
  }
  const uint32_t live = live_tokens(mm, T);

  static_for<KV4>([&](auto it) {
    const int i = tid + kTileThreads * it.value;
    if (i < NK4) {
      const int j = i / (DK / 4), e = (i % (DK / 4)) * 4;
      const bool on = (live >> j) & 1u;
      const f32x4 z = {0.0f, 0.0f, 0.0f, 0.0f};
      *reinterpret_cast<f32x4*>(&Ks[j][e]) = on ? IO<DT>::cvt4(kr[it.value]) : z;
      *reinterpret_cast<f32x4*>(&Qs[j][e]) = on ? IO<DT>::cvt4(qr[it.value]) : z;
    }
  });
  if (tid < TM * kTileRows) {
    const int j = tid / kTileRows;
    Vs[j][tid % kTileRows] = (live >> j) & 1u ? IO<DT>::cvt1(vr) : 0.0f;
  }
  if (tid < TM) {
    const float ea = GF == GF_ANY && p.ga.mode == GDN_GATES_PRE ? 0.0f : exp_fast(al);
    float g, beta;
    gate_transform<GF>(p.ga.mode, gx, gy, ea, db, g, beta);
    const bool on = mm != 0 && tid < T;
    Gs[tid] = on ? g : 1.0f;
    Bs[tid] = on ? beta : 0.0f;
    Ms[tid] = on ? 1 : 0;
  }
  __syncthreads();

  // Coefficients: 4 lanes per pair s <= t < T, numbered densely (pair p of
  // row t is t(t+1)/2 + s, so T = 4 needs one wave), DK/4 channels a lane.
  {
    const int pair = tid >> 2, part = tid & 3;
    int t = 0;
    while (t + 1 < TM && (t + 1) * (t + 2) / 2 <= pair) ++t;
    const int sidx = pair - t * (t + 1) / 2;
    float kk = 0.0f, kq = 0.0f;
    if (t < T && sidx <= t) {
#pragma unroll
      for (int e = part * (DK / 4); e < (part + 1) * (DK / 4); e += 4) {
        const f32x4 ks = *reinterpret_cast<const f32x4*>(&Ks[sidx][e]);
        const f32x4 kt = *reinterpret_cast<const f32x4*>(&Ks[t][e]);
        const f32x4 qt = *reinterpret_cast<const f32x4*>(&Qs[t][e]);
        kk = fmaf(ks.x, kt.x, fmaf(ks.y, kt.y, fmaf(ks.z, kt.z, fmaf(ks.w, kt.w, kk))));
        kq = fmaf(ks.x, qt.x, fmaf(ks.y, qt.y, fmaf(ks.z, qt.z, fmaf(ks.w, qt.w, kq))));
      }
    }
    kk += dpp_f<GDN_DPP_QUAD_XOR1>(kk);
    kk += dpp_f<GDN_DPP_QUAD_XOR2>(kk);
    kq += dpp_f<GDN_DPP_QUAD_XOR1>(kq);
    kq += dpp_f<GDN_DPP_QUAD_XOR2>(kq);
    if (part == 0 && t < T && sidx <= t) {
      float r = 1.0f;
      for (int u = sidx + 1; u <= t; ++u) r *= Gs[u];
      Ckk[t][sidx] = sidx < t ? r * kk : 0.0f;
      Ckq[t][sidx] = r * kq;
    }
    if (tid < TM) {
      float gm = 1.0f;
      for (int u = 0; u <= tid; ++u) gm *= Gs[u];
      Gam[tid] = gm;
    }
  }
  __syncthreads();

  // Per state row: 2T dot products, then the scalar recurrence.
  float a[TM], b[TM];
  static_for<TM>([&](auto tt) {
    constexpr int t = tt.value;
    a[t] = 0.0f;
    b[t] = 0.0f;
    if (t < T) {
      float pa = 0.0f, pb = 0.0f;
#pragma unroll
      for (int i = 0; i < NV; ++i) {
        const f32x4 kx = *reinterpret_cast<const f32x4*>(&Ks[t][i * 32 + c.sub * 4]);
        const f32x4 qx = *reinterpret_cast<const f32x4*>(&Qs[t][i * 32 + c.sub * 4]);
        pa = fmaf(s[4 * i], kx.x, pa);
        pa = fmaf(s[4 * i + 1], kx.y, pa);
        pa = fmaf(s[4 * i + 2], kx.z, pa);
        pa = fmaf(s[4 * i + 3], kx.w, pa);
        pb = fmaf(s[4 * i], qx.x, pb);
        pb = fmaf(s[4 * i + 1], qx.y, pb);
        pb = fmaf(s[4 * i + 2], qx.z, pb);
        pb = fmaf(s[4 * i + 3], qx.w, pb);
      }
      a[t] = sum8(pa);
      b[t] = sum8(pb);
    }
  });
  const int rloc = tid / kLanesPerRow;
  float dl[TM];
  static_for<TM>([&](auto tt) {
    constexpr int t = tt.value;
    dl[t] = 0.0f;
    if (t < T) {
      float u = Vs[t][rloc] - Gam[t] * a[t];
      float yv = Gam[t] * b[t];
      static_for<t>([&](auto ss) { u = fmaf(-Ckk[t][ss.value], dl[ss.value], u); });
      dl[t] = Bs[t] * u;
      static_for<t + 1>([&](auto ss) { yv = fmaf(Ckq[t][ss.value], dl[ss.value], yv); });
      if (Ms[t] == 0) yv = 0.0f;
      if (c.row_ok && c.sub == 0) IO<DT>::store1(p.y, ((c.tok0 + t) * p.Hv + c.hv) * p.Dv + c.dv, yv);
    }
  });
}

// Verify on MFMA (Dk = 128, bf16 q/k).  The 2T dot products of a state row
// (a_t = S k_t, b_t = S q_t) are one matrix product per 16-row wave tile,
// D = A S^T, with A = [k_0 .. k_{TM-1}; q_0 .. q_{TM-1}] (bf16, exact) and the
// fp32 state split as hi + lo bf16 (two passes, ~2^-16 relative per
// product, fp32 accumulation).
//
// Lane (r, g) of a wave (r = lane % 16, g = lane / 16) holds state row
// dv0 + 16 w + r at columns 32 s + 4 g .. +3 and 32 s + 16 + 4 g .. +3
// (s < 4), so one load instruction covers 64 contiguous bytes of 16 rows.
// Those 8 columns are the lane's 8 k-slots of the MFMA B operand for
// k-step s; A is read from LDS in the same column order.  D[m][r] lands in
// lane (r, m / 4): with TM = 4 lanes g = 0 / 1 hold a_0..3 / b_0..3 of row
// r (TM = 8: a in g = 0, 1 and b in g = 2, 3).  The coefficients k_s . k_t
// and k_s . q_t come from the product A K^T (4 MFMAs per wave).
constexpr int kVmRows = 64;  // state rows per workgroup, 16 per wave

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

__device__ __forceinline__ f32x4 mfma_bf16(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// hi = bf16(x) and lo = bf16(x - hi) of 8 floats, as MFMA operands (element
// e of the result is x[e]).  The residual takes hi back from the packed pair.
__device__ __forceinline__ void split8(const f32x4& x0, const f32x4& x1, bf16x8& hi, bf16x8& lo) {
  const uint32_t h[4] = {pk_bf16(x0.x, x0.y), pk_bf16(x0.z, x0.w), pk_bf16(x1.x, x1.y), pk_bf16(x1.z, x1.w)};
  const float v[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
  uint32_t l[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const float r0 = v[2 * k] - __builtin_bit_cast(float, h[k] << 16);
    const float r1 = v[2 * k + 1] - __builtin_bit_cast(float, h[k] & 0xffff0000u);
    l[k] = pk_bf16(r0, r1);
  }
  hi = __builtin_bit_cast(bf16x8, u32x4{h[0], h[1], h[2], h[3]});
  lo = __builtin_bit_cast(bf16x8, u32x4{l[0], l[1], l[2], l[3]});
}

template <int GF, int TM>
__global__ __launch_bounds__(256) void verify_mfma_kernel(const RecParams p) {
  constexpr int DK = 128;
  constexpr int DT = GDN_DTYPE_BF16;
  constexpr int KP = DK + 8;  // padded LDS row (bf16)
  static_assert(2 * TM <= 16, "the k and q rows fill at most one 16-row MFMA tile");
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int lr = lane & 15, lg = lane >> 4;
  const int hv = blockIdx.y, row = blockIdx.z, hk = hv / p.group;
  const int dv0 = blockIdx.x * kVmRows;
  int slot = row;
  if (p.state_index != nullptr) {
    slot = p.state_index[row];
    if (slot < 0 || slot >= p.n_slots) return;  // uniform, before any barrier
  }
  const int T = p.T;  // 1 <= T <= TM on this path
  const int64_t tok0 = static_cast<int64_t>(row) * T;

  __shared__ __align__(16) uint16_t KQ[16][KP];  // k_0..k_{TM-1}, q_0..q_{TM-1}, then zero rows
  __shared__ float Vs[TM][kVmRows];
  // g_t, beta_t (1 and 0 when masked), mask; slot TM is written by the
  // threads tid >= TM and never read
  __shared__ float Gs[TM + 1], Bs[TM + 1];
  __shared__ uint8_t Ms[TM + 1];
  __shared__ float Cf[4][2][TM][TM];  // per wave: r(t,s) k_s.k_t (s < t), r(t,s) k_s.q_t (s <= t)
  // per wave: its 16 state rows, rows padded to 132 floats so that the
  // operand-layout reads (8 rows, one column group) hit 8 distinct banks
  __shared__ __align__(16) float St[4][16][DK + 4];

  // The state rows are issued first, then every token load (all
  // unconditional, with clamped addresses, and none used before the last is
  // issued): loads complete in issue order, so one latency covers them all.
  // The wave's 16 state rows are read as 8 row pairs, one 1 KB load
  // instruction each (lane l: row 2q + l/32, columns 4(l%32)..+3): a read
  // stream of whole rows runs at ~7.3 TB/s, one of 16 rows x 64 bytes per
  // instruction (the MFMA operand layout) at ~5.7.  The rows reach the
  // operand layout through LDS (33 KB a workgroup, so 4 workgroups fit on a
  // CU instead of 8; the read pattern still wins: 13.7 against 14.6 us per
  // launch at B=32, T=4).
  const int rown = dv0 + 16 * wave + lr;
  const int half = lane >> 5, col4 = (lane & 31) * 4;
  f32x4 ld[8];
#pragma unroll
  for (int q = 0; q < 8; ++q) {
    const int rq = min(dv0 + 16 * wave + 2 * q + half, p.Dv - 1);
    const float* src = p.state_in != nullptr
                           ? p.state_in + ((static_cast<int64_t>(slot) * p.Hv + hv) * p.Dv + rq) * DK
                           : kZeroRow;
    ld[q] = __builtin_nontemporal_load((gbl_f32x4*)(src + col4));
  }
  float al, db;
  param_load_raw<GF, DT>(p.ga, hv, al, db);

  const int kq_m = tid >> 4, kq_e = (tid & 15) * 8;  // 16 bytes a thread, row kq_m
  const int kq_t = kq_m < TM ? kq_m : kq_m - TM;
  u32x4 kq;
  {
    const uint16_t* ks = static_cast<const uint16_t*>(kq_m < TM ? p.k : p.q);
    kq = *reinterpret_cast<const u32x4*>(ks + ((tok0 + min(kq_t, T - 1)) * p.Hk + hk) * DK + kq_e);
  }
  constexpr int NVS = (TM * kVmRows + 255) / 256;
  IO<DT>::raw1 vr[NVS];
#pragma unroll
  for (int j = 0; j < NVS; ++j) {
    const int i = min(tid + 256 * j, TM * kVmRows - 1);
    const int t = i / kVmRows, r = i % kVmRows;
    vr[j] = IO<DT>::load1_raw(p.v, ((tok0 + min(t, T - 1)) * p.Hv + hv) * p.Dv + min(dv0 + r, p.Dv - 1));
  }
  // threads tid < TM keep token tid's gates and mask; the others load a
  // valid token too and never use it
  float gx, gy;
  uint8_t mm;
  {
    const int64_t tok = tok0 + min(tid, T - 1);
    gate_load<GF, DT>(p.ga, tok * p.ga.ld + hv, gx, gy);
    // the mask byte of token lane (the same token as tid in wave 0, whose
    // first TM threads use mm), so that every wave can form the live bits
    const int64_t mtok = tok0 + min(static_cast<int>(tid & 63), T - 1);
    const uint8_t* mp = p.mask != nullptr ? p.mask + mtok : &kActive;
    mm = *(gbl_u8*)mp;
  }
  const uint32_t live = live_tokens(mm, T);

  {
    // zero rows past the k and q rows, and a masked token's rows
    const bool keep = kq_m < 2 * TM && kq_t < T && ((live >> kq_t) & 1u);
    *reinterpret_cast<u32x4*>(&KQ[kq_m][kq_e]) =
        u32x4{keep ? kq.x : 0u, keep ? kq.y : 0u, keep ? kq.z : 0u, keep ? kq.w : 0u};
  }
  // every thread stores (no branch the v loads could be sunk into)
  static_assert(TM * kVmRows % 256 == 0, "the v values fill whole passes of the workgroup");
#pragma unroll
  for (int j = 0; j < NVS; ++j) {
    const int i = tid + 256 * j;
    Vs[i / kVmRows][i % kVmRows] = (live >> (i / kVmRows)) & 1u ? IO<DT>::cvt1(vr[j]) : 0.0f;
  }
  {
    // every thread transforms and stores (a use under a branch would have
    // the gate loads sunk into it, behind the first wait)
    const float ea = GF == GF_ANY && p.ga.mode == GDN_GATES_PRE ? 0.0f : exp_fast(al);
    float g, beta;
    gate_transform<GF>(p.ga.mode, gx, gy, ea, db, g, beta);
    const bool on = mm != 0 && tid < T;
    const int slot_g = min(tid, TM);
    Gs[slot_g] = on ? g : 1.0f;
    Bs[slot_g] = on ? beta : 0.0f;
    Ms[slot_g] = on ? 1 : 0;
  }
#pragma unroll
  for (int q = 0; q < 8; ++q) *reinterpret_cast<f32x4*>(&St[wave][2 * q + half][col4]) = ld[q];
  __syncthreads();

  // A fragments (rows of KQ, columns in the state lanes' order)
  bf16x8 a[4];
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    const u32x2 lo4 = *reinterpret_cast<const u32x2*>(&KQ[lr][32 * s + 4 * lg]);
    const u32x2 hi4 = *reinterpret_cast<const u32x2*>(&KQ[lr][32 * s + 16 + 4 * lg]);
    a[s] = __builtin_bit_cast(bf16x8, u32x4{lo4.x, lo4.y, hi4.x, hi4.y});
  }

  // Coefficients: D_kk = A K^T (B = the k rows of A; lane (n, g) holds
  // D_kk[4 g + i][n]), scaled by r(t, s) = prod_{s < u <= t} g_u.
  {
    const bf16x8 zero8 = {};
    f32x4 dkk = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int s = 0; s < 4; ++s) dkk = mfma_bf16(a[s], lr < TM ? a[s] : zero8, dkk);
    if (lr < TM) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int m = 4 * lg + i, sidx = lr;
        const int t = m < TM ? m : m - TM;
        if (m < 2 * TM) {
          float r = 1.0f;
          for (int u = sidx + 1; u <= t; ++u) r *= Gs[u];
          const bool kk = m < TM;
          const bool on = t < T && (kk ? sidx < t : sidx <= t);
          Cf[wave][kk ? 0 : 1][t][sidx] = on ? r * dkk[i] : 0.0f;
        }
      }
    }
  }

  // a_t, b_t of this wave's 16 rows: lane (r, g) takes row r of the buffer
  // at columns 32 s + 4 g..+3 and 32 s + 16 + 4 g..+3 as its B operand
  f32x4 d = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    const f32x4 x0 = *reinterpret_cast<const f32x4*>(&St[wave][lr][32 * s + 4 * lg]);
    const f32x4 x1 = *reinterpret_cast<const f32x4*>(&St[wave][lr][32 * s + 16 + 4 * lg]);
    bf16x8 sh, sl;
    split8(x0, x1, sh, sl);
    d = mfma_bf16(a[s], sh, d);
    d = mfma_bf16(a[s], sl, d);
  }
  // gather a and b of row r into lane (r, 0)
  float av[TM], bv[TM];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    if constexpr (TM == 4) {
      av[i] = d[i];
      bv[i] = __shfl(d[i], lane + 16, 64);
    } else {
      av[i] = d[i];
      av[4 + i] = __shfl(d[i], lane + 16, 64);
      bv[i] = __shfl(d[i], lane + 32, 64);
      bv[4 + i] = __shfl(d[i], lane + 48, 64);
    }
  }
  // Cf was written by this wave only
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

  // the scalar recurrence of the unrolled verify (as in verify_wy_kernel)
  const bool store = lg == 0 && rown < p.Dv;
  float dl[TM];
  float gam = 1.0f;
  static_for<TM>([&](auto tt) {
    constexpr int t = tt.value;
    dl[t] = 0.0f;
    if (t < T) {
      gam *= Gs[t];
      float u = Vs[t][16 * wave + lr] - gam * av[t];
      float yv = gam * bv[t];
      static_for<t>([&](auto ss) { u = fmaf(-Cf[wave][0][t][ss.value], dl[ss.value], u); });
      dl[t] = Bs[t] * u;
      static_for<t + 1>([&](auto ss) { yv = fmaf(Cf[wave][1][t][ss.value], dl[ss.value], yv); });
      if (Ms[t] == 0) yv = 0.0f;
      if (store) IO<DT>::store1(p.y, ((tok0 + t) * p.Hv + hv) * p.Dv + rown, yv);
    }
  });
}

enum KernelKind { K_DECODE = 0, K_TILE = 1, K_VERIFY = 2 };

template <int GF>
int launch_verify_mfma(hipStream_t st, const RecParams& p, int64_t B) {
  const dim3 grid(static_cast<unsigned>((p.Dv + kVmRows - 1) / kVmRows), static_cast<unsigned>(p.Hv),
                  static_cast<unsigned>(B));
  if (p.T <= 4) hipLaunchKernelGGL((verify_mfma_kernel<GF, 4>), grid, dim3(256), 0, st, p);
  else hipLaunchKernelGGL((verify_mfma_kernel<GF, kVerifyMaxT>), grid, dim3(256), 0, st, p);
  return gdn_host::check_launch("gdn_recurrent");
}

template <int DK, int DT, int GF>
int launch_pf(int kind, dim3 grid, dim3 block, hipStream_t st, const RecParams& p) {
  if constexpr (GF != GF_ANY) {
    // the serving step: every option fixed (see DecodeMode)
    const bool dwords = DT == GDN_DTYPE_F32 ||
                        (gdn_host::aligned(p.v, 4) && gdn_host::aligned(p.ga.gx, 4) && gdn_host::aligned(p.ga.gy, 4) &&
                         p.ga.ld % 2 == 0 && p.Hv % 2 == 0 && p.Dv % 2 == 0);
    const bool lean = kind == K_DECODE && p.T == 1 && p.state_in != nullptr && p.state_out != nullptr &&
                      p.y != nullptr && p.mask == nullptr && p.commit_len == nullptr && p.snapshots == nullptr &&
                      dwords;
    if (lean && p.state_index != nullptr) {
      hipLaunchKernelGGL((recurrent_kernel<DK, DT, GF, kDecodeLeanPooled>), grid, block, 0, st, p);
      return gdn_host::check_launch("gdn_recurrent");
    }
    if (lean) {
      hipLaunchKernelGGL((recurrent_kernel<DK, DT, GF, kDecodeLean>), grid, block, 0, st, p);
      return gdn_host::check_launch("gdn_recurrent");
    }
  }
  if (kind == K_VERIFY && p.T <= 4) hipLaunchKernelGGL((verify_wy_kernel<DK, DT, GF, 4>), grid, block, 0, st, p);
  else if (kind == K_VERIFY)
    hipLaunchKernelGGL((verify_wy_kernel<DK, DT, GF, kVerifyMaxT>), grid, block, 0, st, p);
  else if (kind == K_TILE && p.cu_seqlens == nullptr && p.T <= 4)
    hipLaunchKernelGGL((recurrent_tile_kernel<DK, DT, GF, 4>), grid, block, 0, st, p);
  else if (kind == K_TILE && p.cu_seqlens == nullptr && p.T <= 8)
    hipLaunchKernelGGL((recurrent_tile_kernel<DK, DT, GF, 8>), grid, block, 0, st, p);
  else if (kind == K_TILE) hipLaunchKernelGGL((recurrent_tile_kernel<DK, DT, GF, kTileMax>), grid, block, 0, st, p);
  else hipLaunchKernelGGL((recurrent_kernel<DK, DT, GF, kDecodeAny>), grid, block, 0, st, p);
  return gdn_host::check_launch("gdn_recurrent");
}

template <int DK, int DT>
int launch_gf(int gf, int pf, dim3 grid, dim3 block, hipStream_t st, const RecParams& p) {
  // Typed gate formats are built for the Dk = 128 kernels; other head
  // sizes read gates through the runtime-dtype path.
  if constexpr (DK == 128) {
    if (gf == GF_IO_F32) return launch_pf<DK, DT, GF_IO_F32>(pf, grid, block, st, p);
    if (gf == GF_IO_IO) return launch_pf<DK, DT, GF_IO_IO>(pf, grid, block, st, p);
  }
  return launch_pf<DK, DT, GF_ANY>(pf, grid, block, st, p);
}

template <int DK>
int launch_dt(int dt, int gf, int pf, dim3 grid, dim3 block, hipStream_t st, const RecParams& p) {
  switch (dt) {
    case GDN_DTYPE_BF16:
      return launch_gf<DK, GDN_DTYPE_BF16>(gf, pf, grid, block, st, p);
    case GDN_DTYPE_F16:
      return launch_gf<DK, GDN_DTYPE_F16>(gf, pf, grid, block, st, p);
    default:
      return launch_gf<DK, GDN_DTYPE_F32>(gf, pf, grid, block, st, p);
  }
}

int run_recurrent(const gdn_recurrent_args* a) {
  using gdn_host::fail;
  if (a == nullptr) return fail(GDN_ERR_INVALID, "gdn_recurrent: args is NULL");
  if (a->B < 0 || a->T < 0 || a->Hk <= 0 || a->Hv <= 0 || a->Dv <= 0)
    return fail(GDN_ERR_INVALID, "gdn_recurrent: bad sizes B=%lld T=%lld Hk=%lld Hv=%lld Dv=%lld",
                (long long)a->B, (long long)a->T, (long long)a->Hk, (long long)a->Hv,
                (long long)a->Dv);
  if (a->Hv % a->Hk != 0)
    return fail(GDN_ERR_INVALID, "gdn_recurrent: Hv=%lld is not a multiple of Hk=%lld",
                (long long)a->Hv, (long long)a->Hk);
  if (a->Dk != 64 && a->Dk != 128 && a->Dk != 256)
    return fail(GDN_ERR_UNSUPPORTED, "gdn_recurrent: Dk=%lld not built (64, 128, 256)",
                (long long)a->Dk);
  if (a->Hv > 65535 || a->B > 65535 || a->Dv > (1 << 20))
    return fail(GDN_ERR_UNSUPPORTED, "gdn_recurrent: Hv or B above 65535");
  if (!gdn_host::dtype_ok(a->qkv_dtype) || !gdn_host::dtype_ok(a->gate_dtype))
    return fail(GDN_ERR_INVALID, "gdn_recurrent: bad dtype code");
  if (a->gate_mode != GDN_GATES_RAW && a->gate_mode != GDN_GATES_PRE)
    return fail(GDN_ERR_INVALID, "gdn_recurrent: bad gate_mode %d", a->gate_mode);
  if (a->gate_mode == GDN_GATES_RAW &&
      (a->A_log == nullptr || a->dt_bias == nullptr || !gdn_host::dtype_ok(a->param_dtype)))
    return fail(GDN_ERR_INVALID, "gdn_recurrent: raw gates need A_log, dt_bias and their dtype");
  // With no tokens the launch only copies state_in to state_out, and empty
  // token tensors may legitimately come with NULL data pointers.
  if (a->T > 0 && (a->k == nullptr || a->v == nullptr || a->gx == nullptr || a->gy == nullptr))
    return fail(GDN_ERR_INVALID, "gdn_recurrent: k, v and gates are required");
  if (a->T > 0 && a->y != nullptr && a->q == nullptr)
    return fail(GDN_ERR_INVALID, "gdn_recurrent: q is required when y is requested");
  const size_t el = a->qkv_dtype == GDN_DTYPE_F32 ? 16 : 8;
  if (!gdn_host::aligned(a->q, el) || !gdn_host::aligned(a->k, el) ||
      !gdn_host::aligned(a->state_in, 16) || !gdn_host::aligned(a->state_out, 16) ||
      !gdn_host::aligned(a->snapshots, 16))
    return fail(GDN_ERR_INVALID, "gdn_recurrent: q/k or state pointers are misaligned");
  if (a->gate_stride != 0 && a->gate_stride < a->Hv)
    return fail(GDN_ERR_INVALID, "gdn_recurrent: gate_stride=%lld is below Hv=%lld", (long long)a->gate_stride,
                (long long)a->Hv);
  if (a->state_index != nullptr && (a->n_slots < 0 || a->n_slots > INT32_MAX))
    return fail(GDN_ERR_INVALID, "gdn_recurrent: n_slots=%lld out of range", (long long)a->n_slots);
  if (a->y_from < 0 || (a->y_from > 0 && (a->y == nullptr || a->y_from > a->T)))
    return fail(GDN_ERR_INVALID, "gdn_recurrent: y_from=%lld must be in [0, T] and needs y", (long long)a->y_from);
  if (a->B == 0) return GDN_OK;
  if (a->T > INT32_MAX) return fail(GDN_ERR_UNSUPPORTED, "gdn_recurrent: T too large");

  RecParams p;
  p.q = a->q;
  p.k = a->k;
  p.v = a->v;
  p.ga.gx = a->gx;
  p.ga.gy = a->gy;
  p.ga.ld = a->gate_stride > 0 ? a->gate_stride : a->Hv;
  p.ga.A_log = a->A_log;
  p.ga.dt_bias = a->dt_bias;
  p.ga.mode = a->gate_mode;
  p.ga.gdt = a->gate_dtype;
  p.ga.pdt = a->param_dtype;
  p.state_in = a->state_in;
  p.state_out = a->state_out;
  p.snapshots = a->snapshots;
  p.y = a->y;
  p.mask = a->mask;
  p.cu_seqlens = a->cu_seqlens;
  p.commit_len = a->commit_len;
  p.y_from = static_cast<int>(a->y_from);
  p.state_index = a->state_index;
  p.n_slots = a->state_index != nullptr ? static_cast<int>(a->n_slots) : 0;
  p.T = static_cast<int>(a->T);
  p.Hk = static_cast<int>(a->Hk);
  p.Hv = static_cast<int>(a->Hv);
  p.Dv = static_cast<int>(a->Dv);
  p.group = static_cast<int>(a->Hv / a->Hk);
  // hv / group = (hv * ceil(2^31 / group)) >> 31 exactly while hv * group <= 2^31
  // (hv < 2^16, and the decode kernel is only used for group < 2^15)
  p.group_magic = static_cast<unsigned>(((1ull << 31) + p.group - 1) / p.group);

  int gf = GF_ANY;
  if (a->gate_mode == GDN_GATES_RAW && a->gate_dtype == a->qkv_dtype) {
    if (a->param_dtype == GDN_DTYPE_F32) gf = GF_IO_F32;
    else if (a->param_dtype == a->qkv_dtype) gf = GF_IO_IO;
  }

  // Waves per workgroup: the largest of 4/2/1 that still gives >= 1024
  // workgroups (4 per CU), so small batches spread over the 256 CUs.
  // Tokens per row > 1 (or packed rows): stage token tiles in LDS, with
  // workgroups of 4 waves.
  // A verify of a few tokens without state writes or snapshots: the
  // unrolled form (verify_wy_kernel), same 32-row workgroups.
  // (y_from > 0 takes the tile kernel: only it leaves tokens without y)
  const bool verify = a->state_out == nullptr && a->snapshots == nullptr && a->y != nullptr &&
                      a->cu_seqlens == nullptr && a->commit_len == nullptr && a->T >= 1 &&
                      a->T <= kVerifyMaxT && a->y_from == 0;
  // The decode kernel indexes in 32 bits: state rows (pool slots or B, times
  // Hv*Dv), q/k/v/y elements and gate entries must stay below 2^31 (and the
  // group below 2^15, for its division); larger launches take the tile
  // kernel, whose steps are bit-identical.
  const int64_t state_rows = (a->state_index != nullptr ? a->n_slots : a->B) * a->Hv * a->Dv;
  const bool idx32 = state_rows < (int64_t{1} << 31) && a->B * a->Hv * a->Dv < (int64_t{1} << 31) &&
                     a->B * a->Hk * a->Dk < (int64_t{1} << 31) && a->B * p.ga.ld < (int64_t{1} << 31) &&
                     p.group < (1 << 15);
  const bool pf = a->T > 1 || a->cu_seqlens != nullptr || !idx32 || a->y_from > 0;
  const int kind = verify ? K_VERIFY : (pf ? K_TILE : K_DECODE);
  // the tile and verify kernels assume workgroups of 4 waves (32 rows)
  const bool four = kind != K_DECODE;
  // state rows per wave: 8 in the tile and verify kernels, 256/Dk in the
  // decode kernel (Dk/4 lanes per row)
  const int rows_per_wave = four ? 8 : static_cast<int>(256 / a->Dk);
  int waves = four ? 4 : 1;
  for (int w = 4; w >= 1 && !four; w >>= 1) {
    const int64_t rows_per_wg = rows_per_wave * w;
    const int64_t wgs = a->B * a->Hv * ((a->Dv + rows_per_wg - 1) / rows_per_wg);
    if (wgs >= 1024 || w == 1) {
      waves = w;
      break;
    }
  }
  const int rows_per_wg = rows_per_wave * waves;
  p.wg_rows = rows_per_wg;
  dim3 block(64 * waves);
  dim3 grid(static_cast<unsigned>((a->Dv + rows_per_wg - 1) / rows_per_wg),
            static_cast<unsigned>(a->Hv), static_cast<unsigned>(a->B));
  hipStream_t st = static_cast<hipStream_t>(a->stream);
  // bf16 q/k at Dk = 128 (16-byte aligned rows): the verify's dot products
  // on MFMA (verify_mfma_kernel, 64-row workgroups)
  if (kind == K_VERIFY && a->Dk == 128 && a->qkv_dtype == GDN_DTYPE_BF16 && gdn_host::aligned(a->q, 16) &&
      gdn_host::aligned(a->k, 16)) {
    if (gf == GF_IO_F32) return launch_verify_mfma<GF_IO_F32>(st, p, a->B);
    if (gf == GF_IO_IO) return launch_verify_mfma<GF_IO_IO>(st, p, a->B);
    return launch_verify_mfma<GF_ANY>(st, p, a->B);
  }
  switch (a->Dk) {
    case 64:
      return launch_dt<64>(a->qkv_dtype, gf, kind, grid, block, st, p);
    case 128:
      return launch_dt<128>(a->qkv_dtype, gf, kind, grid, block, st, p);
    default:
      return launch_dt<256>(a->qkv_dtype, gf, kind, grid, block, st, p);
  }
}

}  // namespace

extern "C" int gdn_recurrent(const gdn_recurrent_args* args) { return run_recurrent(args); }

extern "C" int gdn_gated_delta_update(const void* q, const void* k, const void* v, int qkv_dtype,
                                      const void* a, const void* b, int ab_dtype,
                                      const void* A_log, const void* dt_bias, int param_dtype,
                                      const float* state_in, const uint8_t* mask, void* y,
                                      float* state_out, int64_t B, int64_t T, int64_t Hk,
                                      int64_t Hv, int64_t Dk, int64_t Dv, void* stream) {
  if (state_out == nullptr || (T > 0 && (y == nullptr || q == nullptr)))
    return gdn_host::fail(GDN_ERR_INVALID, "gdn_gated_delta_update: q, y and state_out are required");
  gdn_recurrent_args r = {};
  r.q = q;
  r.k = k;
  r.v = v;
  r.qkv_dtype = qkv_dtype;
  r.gate_mode = GDN_GATES_RAW;
  r.gx = a;
  r.gy = b;
  r.gate_dtype = ab_dtype;
  r.param_dtype = param_dtype;
  r.A_log = A_log;
  r.dt_bias = dt_bias;
  r.state_in = state_in;
  r.state_out = state_out;
  r.y = y;
  r.mask = mask;
  r.B = B;
  r.T = T;
  r.Hk = Hk;
  r.Hv = Hv;
  r.Dk = Dk;
  r.Dv = Dv;
  r.stream = stream;
  return run_recurrent(&r);
}

extern "C" int gdn_gated_delta_kernel(const void* q, const void* k, const void* v, int qkv_dtype,
                                      const void* g, const void* beta, int gb_dtype,
                                      const float* state_in, const uint8_t* mask, void* y,
                                      float* state_out, int64_t B, int64_t T, int64_t Hk,
                                      int64_t Hv, int64_t Dk, int64_t Dv, void* stream) {
  if (state_out == nullptr || (T > 0 && (y == nullptr || q == nullptr)))
    return gdn_host::fail(GDN_ERR_INVALID, "gdn_gated_delta_kernel: q, y and state_out are required");
  gdn_recurrent_args r = {};
  r.q = q;
  r.k = k;
  r.v = v;
  r.qkv_dtype = qkv_dtype;
  r.gate_mode = GDN_GATES_PRE;
  r.gx = g;
  r.gy = beta;
  r.gate_dtype = gb_dtype;
  r.param_dtype = GDN_DTYPE_F32;
  r.state_in = state_in;
  r.state_out = state_out;
  r.y = y;
  r.mask = mask;
  r.B = B;
  r.T = T;
  r.Hk = Hk;
  r.Hv = Hv;
  r.Dk = Dk;
  r.Dv = Dv;
  r.stream = stream;
  return run_recurrent(&r);
}
