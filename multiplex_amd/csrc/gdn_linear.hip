// Decode-shape projections of the GatedDeltaNet mixer on gfx950 bf16 MFMA:
//
//   out[M, N] = A[M, K] W[N, K]^T,   M <= 64 rows (one token per decoding row),
//
// where A is either the input rows (in_proj, dflash.py:348-350) or the
// mixer epilogue's gated RMSNorm of the GDN output computed on the fly
// (norm(out, z) then out_proj, dflash.py:377-378):
//
//   A[r, h*hd + c] = bf16( round(w[c] round(y[r, h*hd + c] * rsq)) * silu(z[r, h*hd + c]) ),
//   rsq = 1 / sqrt(mean_c y[r, h*hd + c]^2 + eps)   over each head of hd columns,
//
// with gdn_gated_rmsnorm's rounding points.
//
// At decode the weights dominate the bytes (out_proj 16 MiB, in_proj 48 MiB
// at hidden 2048) and A is small but read against every weight column.  The
// grid splits N into 64-column tiles and K into 512-wide slices: one
// workgroup per (tile, slice), each wave one 128-wide quarter of the slice,
// reads its W rows once and its A rows once, both straight into MFMA
// registers, every load issued before the first wait.  A workgroup covers
// as few 16-row blocks as hold M (1, 2 or 4), so small batches use fewer
// registers and less LDS and more workgroups share a CU.  The waves' partial
// tiles are summed in LDS and go to an fp32 workspace; the last workgroup of
// a tile to finish sums the slices in slice order (so the result does not
// depend on which finished last), writes the bf16 tile and resets the tile's
// ticket.
//
// Measured against hipBLASLt (graph-replayed, out_proj 4096 -> 2048): with
// the norm fused it beats the separate norm plus the library GEMM up to 16
// rows (7.4-8.1 us against 12.6-13.4 us) and loses beyond (at 64 rows every
// workgroup re-reads y and z for its K slice, twice the weight bytes it
// streams); the plain projection never beats the library.  Callers dispatch
// on that.
//
// The slices of one tile meet without fences.  Each workgroup writes its
// partial tile with device-coherent stores (cache policy sc1, the encoding
// of an agent-scope store: not held back in the writer's L2) and waits for
// them to complete before it takes the tile's ticket; the last workgroup
// reads the partials with device-coherent loads (sc1).  So the sum is right
// whichever XCDs the slices run on.  The grid still deals every slice of a
// tile to one XCD by block index (block b normally runs on XCD b % 8), but
// the hardware does not always keep to that: the XCC_ID register has shown
// blocks of other kernels off that XCD in about one launch in seven.  No
// workgroup waits for another.
#include "gdn_common.hpp"

namespace {

using namespace gdn;

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int LM = 64;        // most rows per launch
constexpr int LN = 64;        // output columns per workgroup
constexpr int LK = 512;       // K per workgroup
constexpr int kXcds = 8;

struct LinParams {
  const uint16_t* x;  // A rows, or the GDN output y when norming
  int64_t ldx;
  const uint16_t* g;  // the norm's gate z (NORM)
  int64_t ldg;
  const void* nw;     // the norm's weight [hd] (NORM; null = ones)
  float eps;
  const uint16_t* w;  // W [N, K]
  uint16_t* out;
  int64_t ldo;
  float* part;        // [KSL][16 MB][NT * LN] fp32 partial sums
  uint32_t* tickets;  // [NT], at the start of the workspace
  int M, N, K, NT, KSL;
};

__device__ __forceinline__ f32x4 mfma16(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ bf16x8 ld_bf16x8(const uint16_t* p) {
  return __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4*>(p));
}

__device__ __forceinline__ float round_bf16(float x) { return bf16_to_f32(f32_to_bf16(x)); }

// Sum over the four 16-lane rows of a wave (lanes l, l + 16, l + 32, l + 48),
// by the gfx950 row swaps: permlane16_swap(x, x) yields the even and the odd
// rows, permlane32_swap the low and the high halves, each in both places.
__device__ __forceinline__ float rows_sum4(float x) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

typedef __amdgpu_buffer_rsrc_t BufRsrc;
constexpr int kBufFlags = 0x00020000;  // raw buffer, 32-bit data format (gfx9)
constexpr int kDeviceCoherent = 16;   // cache policy sc1: the access is coherent across the device's XCDs

// out^T (64 columns x 64 rows) += W A^T over one wave's k-steps, into this
// wave's slot of the LDS reduction buffer: accumulator (mb, nb) lane (lr, lq)
// holds out^T[16 nb + 4 lq + i][16 mb + lr], i.e. out[16 mb + lr][16 nb + 4 lq + i].
template <int MB, int NB, int SQ>
__device__ __forceinline__ void mma_tile(const bf16x8 (&af)[MB][SQ], const bf16x8 (&wf)[NB][SQ],
                                         float (&slot)[MB][NB][64][4], int lane) {
  f32x4 acc[MB][NB];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb)
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) acc[mb][nb] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int s = 0; s < SQ; ++s)
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) acc[mb][nb] = mfma16(wf[nb][s], af[mb][s], acc[mb][nb]);
#pragma unroll
  for (int mb = 0; mb < MB; ++mb)
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) *reinterpret_cast<f32x4*>(slot[mb][nb][lane]) = acc[mb][nb];
}

// NORM: A is the gated RMSNorm of y (heads of HD columns, weight dtype WT).
//
// Wave w takes the K quarter [k0 + 128 w, k0 + 128 w + 128) of the slice --
// one head at HD = 128 -- for the whole 64 x 64 tile, so neither operand
// goes through LDS: its A rows (normalised in registers when NORM) and its W
// rows are MFMA fragments as loaded.  A is loaded first (it comes from the
// L2), so the norm's arithmetic overlaps the W rows' trip from HBM.  The
// four waves' partial tiles are then summed once in LDS.
//
// One wave per SIMD (waves_per_eu 1): the wave may hold all of its operands
// at once, so every load is issued before the first wait; with the default
// budget of 128 registers the compiler splits them into batches, one memory
// round trip each.
template <bool NORM, int HD, int WT, int MB>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(MB == 4 ? 1 : 2))) void
linear_decode_kernel(const LinParams p) {
  constexpr int KQ = LK / 4;      // K per wave (128)
  constexpr int SQ = KQ / 32;     // k-steps per wave (4)
  constexpr int RM = 16 * MB;     // rows this launch covers
  constexpr int NB = LN / 16;     // column blocks (4)
  static_assert(!NORM || (HD <= KQ && KQ % HD == 0), "a head lies within one wave's quarter");
  const int blk = blockIdx.x;
  const int xcd = blk % kXcds, r8 = blk / kXcds;
  const int ks = r8 % p.KSL;
  const int nt = (r8 / p.KSL) * kXcds + xcd;  // all slices of tile nt on XCD nt % 8
  if (nt >= p.NT) return;                     // grid padding (uniform, before any barrier)
  const int n0 = nt * LN;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lr = lane & 15, lq = lane >> 4, lg8 = lq * 8;
  const int kw = ks * LK + wave * KQ;  // this wave's first column

  __shared__ __align__(16) float red[4][MB][NB][64][4];  // each wave's partial tile, lane-major
  __shared__ int s_last;

  // A fragments (B operand of out^T = W A^T): rows 16 mb + lr, columns kw + 32 s + 8 lq ..
  // (rows past M re-read row M-1; their sums are never stored)
  bf16x8 af[MB][SQ];
  if constexpr (NORM) {
    // the norm weight over this wave's columns within its head (a null
    // weight reads as ones: the loads then read y's first row, unused)
    const bool has_w = p.nw != nullptr;
    Raw8<WT> raw[SQ];
#pragma unroll
    for (int s = 0; s < SQ; ++s) raw[s] = load_raw8<WT>(has_w ? p.nw : p.x, (wave * KQ + 32 * s + lg8) % HD);
    u32x4 xr[MB][SQ], gr[MB][SQ];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
      const int r = min(16 * mb + lr, p.M - 1);
#pragma unroll
      for (int s = 0; s < SQ; ++s) {
        xr[mb][s] = *reinterpret_cast<const u32x4*>(p.x + static_cast<int64_t>(r) * p.ldx + kw + 32 * s + lg8);
        gr[mb][s] = *reinterpret_cast<const u32x4*>(p.g + static_cast<int64_t>(r) * p.ldg + kw + 32 * s + lg8);
      }
    }
    // W rows after A: the norm below waits for A only (loads complete in order)
    bf16x8 wf[NB][SQ];
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
      const int n = min(n0 + 16 * nb + lr, p.N - 1);
#pragma unroll
      for (int s = 0; s < SQ; ++s) wf[nb][s] = ld_bf16x8(p.w + static_cast<int64_t>(n) * p.K + kw + 32 * s + lg8);
    }
    __builtin_amdgcn_sched_barrier(0);  // every load above is issued before the first wait below
    float wv[SQ][8];
#pragma unroll
    for (int s = 0; s < SQ; ++s) {
      unpack8<WT>(raw[s], wv[s]);
#pragma unroll
      for (int e = 0; e < 8; ++e) wv[s][e] = has_w ? wv[s][e] : 1.0f;
    }
    constexpr int QPH = HD / 32 < SQ ? HD / 32 : SQ;  // k-steps per head within the quarter
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
      float xv[SQ][8], gv[SQ][8];
#pragma unroll
      for (int s = 0; s < SQ; ++s) {
        unpack8<GDN_DTYPE_BF16>(Raw8<GDN_DTYPE_BF16>{xr[mb][s]}, xv[s]);
        unpack8<GDN_DTYPE_BF16>(Raw8<GDN_DTYPE_BF16>{gr[mb][s]}, gv[s]);
      }
#pragma unroll
      for (int h0 = 0; h0 < SQ; h0 += QPH) {
        float ss = 0.0f;
#pragma unroll
        for (int s = h0; s < h0 + QPH; ++s)
#pragma unroll
          for (int e = 0; e < 8; ++e) ss += xv[s][e] * xv[s][e];
        ss = rows_sum4(ss);  // over the 4 lanes of the row: all of the head's columns
        const float rs = rsqrtf(ss * (1.0f / HD) + p.eps);
#pragma unroll
        for (int s = h0; s < h0 + QPH; ++s) {
          float o[8];
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const float nv = round_bf16(xv[s][e] * rs);
            const float m = (has_w && WT == GDN_DTYPE_BF16) ? round_bf16(wv[s][e] * nv) : wv[s][e] * nv;
            o[e] = m * silu(gv[s][e]);
          }
          af[mb][s] = __builtin_bit_cast(
              bf16x8, u32x4{pk_bf16(o[0], o[1]), pk_bf16(o[2], o[3]), pk_bf16(o[4], o[5]), pk_bf16(o[6], o[7])});
        }
      }
    }
    mma_tile<MB, NB, SQ>(af, wf, red[wave], lane);
  } else {
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
      const int r = min(16 * mb + lr, p.M - 1);
#pragma unroll
      for (int s = 0; s < SQ; ++s) af[mb][s] = ld_bf16x8(p.x + static_cast<int64_t>(r) * p.ldx + kw + 32 * s + lg8);
    }
    bf16x8 wf[NB][SQ];
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
      const int n = min(n0 + 16 * nb + lr, p.N - 1);
#pragma unroll
      for (int s = 0; s < SQ; ++s) wf[nb][s] = ld_bf16x8(p.w + static_cast<int64_t>(n) * p.K + kw + 32 * s + lg8);
    }
    __builtin_amdgcn_sched_barrier(0);  // every load above is issued before the first wait
    mma_tile<MB, NB, SQ>(af, wf, red[wave], lane);
  }
  __syncthreads();

  // The workgroup's partial tile: wave w sums the four waves' blocks w,
  // w + 4, .. of the MB x NB and stores them (lane (lr, lq) of block
  // (mb, nb) holds out[16 mb + lr][n0 + 16 nb + 4 lq + i]).
  const int64_t prow = static_cast<int64_t>(p.NT) * LN;  // partial row stride (floats)
  const BufRsrc pr = __builtin_amdgcn_make_buffer_rsrc(
      p.part, 0, static_cast<int>(static_cast<int64_t>(p.KSL) * RM * prow * 4), kBufFlags);
#pragma unroll
  for (int b = wave; b < MB * NB; b += 4) {
    const int mb = b / NB, nb = b % NB;
    f32x4 sum = *reinterpret_cast<const f32x4*>(red[0][mb][nb][lane]);
#pragma unroll
    for (int w = 1; w < 4; ++w) sum += *reinterpret_cast<const f32x4*>(red[w][mb][nb][lane]);
    const uint32_t off = static_cast<uint32_t>(((ks * RM + 16 * mb + lr) * prow + n0 + 16 * nb + 4 * lq) * 4);
    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, sum), pr, off, 0, kDeviceCoherent);
  }

  // every partial store of this workgroup complete before its ticket
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (tid == 0) s_last = atomicAdd(&p.tickets[nt], 1u) == static_cast<uint32_t>(p.KSL - 1);
  __syncthreads();
  if (!s_last) return;
  if (tid == 0) atomicExch(&p.tickets[nt], 0u);  // ready for the next launch

  // Sum the slices in slice order: thread tid takes quads (row, 4 columns).
#pragma unroll
  for (int q = 0; q < (RM * LN / 4 + 255) / 256; ++q) {
    const int idx = tid + 256 * q;
    const int row = idx / (LN / 4), c = (idx % (LN / 4)) * 4;
    if (row >= p.M || n0 + c >= p.N) continue;
    f32x4 sum = {0.0f, 0.0f, 0.0f, 0.0f};
    const uint32_t off = static_cast<uint32_t>((row * prow + n0 + c) * 4);
    // eight slices' loads in flight before the first add
    for (int k0 = 0; k0 < p.KSL; k0 += 8) {
      f32x4 v[8];
#pragma unroll
      for (int k = 0; k < 8; ++k)
        if (k0 + k < p.KSL)
          v[k] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                               pr, off + static_cast<uint32_t>((k0 + k) * RM * prow * 4), 0,
                                               kDeviceCoherent));
#pragma unroll
      for (int k = 0; k < 8; ++k)
        if (k0 + k < p.KSL) sum += v[k];
    }
    *reinterpret_cast<u32x2*>(p.out + row * p.ldo + n0 + c) = u32x2{pk_bf16(sum[0], sum[1]), pk_bf16(sum[2], sum[3])};
  }
}

// Row blocks per workgroup: 16-row blocks, as few as cover M, so small
// batches hold fewer registers and less LDS and more workgroups share a CU.
int row_blocks(int64_t M) { return M <= 16 ? 1 : M <= 32 ? 2 : 4; }
int64_t n_tiles(int64_t N) { return (N + LN - 1) / LN; }
size_t part_floats(int64_t M, int64_t N, int64_t K) {
  return static_cast<size_t>(K / LK) * 16 * row_blocks(M) * n_tiles(N) * LN;
}

// The workspace starts with a ticket region of fixed size, so calls of
// different shapes that share one workspace never write partial sums over
// each other's tickets (every call leaves its tickets zero).
constexpr int64_t kMaxTiles = 4096;
constexpr int64_t kMaxN = kMaxTiles * LN;
constexpr size_t kTicketBytes = kMaxTiles * 4;

template <int MB>
void launch(const LinParams& p, bool norm, int64_t head_dim, bool wf32, dim3 grid, hipStream_t st) {
  if (!norm) {
    hipLaunchKernelGGL((linear_decode_kernel<false, 128, GDN_DTYPE_BF16, MB>), grid, dim3(256), 0, st, p);
  } else if (head_dim == 64) {
    if (wf32) hipLaunchKernelGGL((linear_decode_kernel<true, 64, GDN_DTYPE_F32, MB>), grid, dim3(256), 0, st, p);
    else hipLaunchKernelGGL((linear_decode_kernel<true, 64, GDN_DTYPE_BF16, MB>), grid, dim3(256), 0, st, p);
  } else {
    if (wf32) hipLaunchKernelGGL((linear_decode_kernel<true, 128, GDN_DTYPE_F32, MB>), grid, dim3(256), 0, st, p);
    else hipLaunchKernelGGL((linear_decode_kernel<true, 128, GDN_DTYPE_BF16, MB>), grid, dim3(256), 0, st, p);
  }
}

}  // namespace

extern "C" size_t gdn_linear_decode_workspace_bytes(int64_t M, int64_t N, int64_t K) {
  if (M < 1 || M > LM || N < 1 || N > kMaxN || K < LK || K % LK != 0) return 0;
  return kTicketBytes + part_floats(M, N, K) * 4;
}

extern "C" int gdn_linear_decode(const void* x, int64_t ldx, const void* gate, int64_t ldg, const void* norm_w,
                                 int norm_w_dtype, float eps, int64_t head_dim, const void* W, void* out,
                                 int64_t ldo, int64_t M, int64_t N, int64_t K, void* workspace,
                                 size_t workspace_bytes, void* stream) {
  using gdn_host::fail;
  if (M < 1 || M > LM) return fail(GDN_ERR_UNSUPPORTED, "gdn_linear_decode: M=%lld outside [1, %d]", (long long)M, LM);
  if (K < LK || K % LK != 0)
    return fail(GDN_ERR_UNSUPPORTED, "gdn_linear_decode: K=%lld is not a multiple of %d", (long long)K, LK);
  if (N < 1 || N % 8 != 0 || N > kMaxN)
    return fail(GDN_ERR_UNSUPPORTED, "gdn_linear_decode: N=%lld must be a positive multiple of 8 up to %lld",
                (long long)N, (long long)kMaxN);
  if (!x || !W || !out || !workspace) return fail(GDN_ERR_INVALID, "gdn_linear_decode: null pointer");
  const bool norm = gate != nullptr;
  if (ldx < K || ldo < N || ldx % 8 != 0 || ldo % 8 != 0 || (norm && (ldg < K || ldg % 8 != 0)))
    return fail(GDN_ERR_INVALID, "gdn_linear_decode: row strides must cover the rows and be multiples of 8");
  if (norm && head_dim != 64 && head_dim != 128)
    return fail(GDN_ERR_UNSUPPORTED, "gdn_linear_decode: head_dim must be 64 or 128");
  if (norm && norm_w != nullptr && norm_w_dtype != GDN_DTYPE_BF16 && norm_w_dtype != GDN_DTYPE_F32)
    return fail(GDN_ERR_INVALID, "gdn_linear_decode: the norm weight must be bf16 or fp32");
  if (norm && !(eps >= 0.0f)) return fail(GDN_ERR_INVALID, "gdn_linear_decode: eps must be >= 0");
  const size_t need = gdn_linear_decode_workspace_bytes(M, N, K);
  if (workspace_bytes < need)
    return fail(GDN_ERR_INVALID, "gdn_linear_decode: workspace of %zu bytes is below the %zu needed",
                workspace_bytes, need);
  if (!gdn_host::aligned(x, 16) || !gdn_host::aligned(W, 16) || !gdn_host::aligned(out, 16) ||
      !gdn_host::aligned(gate, 16) || !gdn_host::aligned(norm_w, 16) || !gdn_host::aligned(workspace, 16))
    return fail(GDN_ERR_INVALID, "gdn_linear_decode: pointers must be 16-byte aligned");
  const int64_t nt = n_tiles(N), ksl = K / LK;
  if (part_floats(M, N, K) * 4 > static_cast<size_t>(INT32_MAX))
    return fail(GDN_ERR_UNSUPPORTED, "gdn_linear_decode: problem too large");

  LinParams p;
  p.x = static_cast<const uint16_t*>(x);
  p.ldx = ldx;
  p.g = static_cast<const uint16_t*>(gate);
  p.ldg = ldg;
  p.nw = norm_w;
  p.eps = eps;
  p.w = static_cast<const uint16_t*>(W);
  p.out = static_cast<uint16_t*>(out);
  p.ldo = ldo;
  p.tickets = static_cast<uint32_t*>(workspace);
  p.part = reinterpret_cast<float*>(static_cast<unsigned char*>(workspace) + kTicketBytes);
  p.M = static_cast<int>(M);
  p.N = static_cast<int>(N);
  p.K = static_cast<int>(K);
  p.NT = static_cast<int>(nt);
  p.KSL = static_cast<int>(ksl);
  const dim3 grid(static_cast<unsigned>((nt + kXcds - 1) / kXcds * kXcds * ksl));
  hipStream_t st = static_cast<hipStream_t>(stream);
  const bool wf32 = norm_w_dtype == GDN_DTYPE_F32;
  switch (row_blocks(M)) {
    case 1: launch<1>(p, norm, head_dim, wf32, grid, st); break;
    case 2: launch<2>(p, norm, head_dim, wf32, grid, st); break;
    default: launch<4>(p, norm, head_dim, wf32, grid, st); break;
  }
  return gdn_host::check_launch("gdn_linear_decode");
}
