// Gated RMSNorm of the GatedDeltaNet mixer epilogue (the `norm(out, z)` call
// at dflash.py:377): per row of D channels,
//   n = x / sqrt(mean(x^2) + eps),  m = w * n,  out = m * silu(gate).
// Bound by HBM: x and gate are read once and out written once, 3 x D x
// sizeof(io) bytes per row; the weight row stays in cache.
//
// A lane owns 8 adjacent channels (one 16-byte access of a bf16 row), so a
// row spans D/8 lanes and the sum of squares is a DPP reduction over them.
// Rounding follows Qwen3NextRMSNormGated (transformers,
// models/qwen3_next/modeling_qwen3_next.py:57-74): n is rounded to the io
// dtype; m is rounded to it too when the weight has the io dtype (a product
// of two half-precision tensors), not when the weight is fp32; the gate
// product is formed in fp32 and rounded once at the store.
#include "gdn_common.hpp"

namespace {

using namespace gdn;

constexpr int kThreads = 256;

template <int DT>
__device__ __forceinline__ float round_io(float x) {
  if constexpr (DT == GDN_DTYPE_BF16) return bf16_to_f32(f32_to_bf16(x));
  else if constexpr (DT == GDN_DTYPE_F16) return f16_to_f32(f32_to_f16(x));
  else return x;
}

// HAS_W: a weight row is given (else the weight is 1).  WT: its dtype.
// Gate row r lies at (r / group) * ld + (r % group) * D: group rows of D
// channels per gate line (a token's heads) with lines ld elements apart.
template <int D, int DT, int WT, bool HAS_W>
__global__ __launch_bounds__(kThreads) void gated_rmsnorm_kernel(const void* x,
                                                                 const void* gate,
                                                                 const void* __restrict__ w, void* out,
                                                                 int64_t rows, int group, int64_t ld,
                                                                 float eps) {
  constexpr int LPR = D / CPL;            // lanes per row
  constexpr int RPB = kThreads / LPR;     // rows per workgroup
  const int sub = threadIdx.x % LPR;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * RPB + threadIdx.x / LPR;
  const bool active = row < rows;
  // A lane group past the last row reads row 0 (rows >= 1) and stores
  // nothing; its lanes still take part in their own group's reduction.
  const int rr = active ? static_cast<int>(row) : 0;  // rows <= INT32_MAX
  const int64_t i = static_cast<int64_t>(rr) * D + sub * CPL;
  const int64_t gi = static_cast<int64_t>(rr / group) * ld + (rr % group) * D + sub * CPL;

  float xv[CPL], gv[CPL], wv[CPL];
  unpack8<DT>(load_raw8<DT>(x, i), xv);
  unpack8<DT>(load_raw8<DT>(gate, gi), gv);
  if constexpr (HAS_W) {
    unpack8<WT>(load_raw8<WT>(w, sub * CPL), wv);
  } else {
#pragma unroll
    for (int k = 0; k < CPL; ++k) wv[k] = 1.0f;
  }
  float ss = 0.0f;
#pragma unroll
  for (int k = 0; k < CPL; ++k) ss += xv[k] * xv[k];
  ss = head_sum<LPR>(ss);
  const float r = rsqrtf(ss * (1.0f / D) + eps);

  float o[CPL];
#pragma unroll
  for (int k = 0; k < CPL; ++k) {
    const float n = round_io<DT>(xv[k] * r);
    const float m = (HAS_W && WT == DT) ? round_io<DT>(wv[k] * n) : wv[k] * n;
    o[k] = m * silu(gv[k]);
  }
  if (active) store8<DT>(out, i, o);
}

template <int D, int DT>
void launch_norm(dim3 grid, hipStream_t st, const void* x, const void* gate, const void* w, int w_dtype,
                 void* out, int64_t rows, int group, int64_t ld, float eps) {
  if (w == nullptr) {
    hipLaunchKernelGGL((gated_rmsnorm_kernel<D, DT, DT, false>), grid, dim3(kThreads), 0, st, x, gate, w, out,
                       rows, group, ld, eps);
  } else if (w_dtype == GDN_DTYPE_F32) {
    hipLaunchKernelGGL((gated_rmsnorm_kernel<D, DT, GDN_DTYPE_F32, true>), grid, dim3(kThreads), 0, st, x, gate,
                       w, out, rows, group, ld, eps);
  } else if (w_dtype == GDN_DTYPE_BF16) {
    hipLaunchKernelGGL((gated_rmsnorm_kernel<D, DT, GDN_DTYPE_BF16, true>), grid, dim3(kThreads), 0, st, x, gate,
                       w, out, rows, group, ld, eps);
  } else {
    hipLaunchKernelGGL((gated_rmsnorm_kernel<D, DT, GDN_DTYPE_F16, true>), grid, dim3(kThreads), 0, st, x, gate,
                       w, out, rows, group, ld, eps);
  }
}

template <int D>
void launch_norm_dt(int io_dtype, dim3 grid, hipStream_t st, const void* x, const void* gate, const void* w,
                    int w_dtype, void* out, int64_t rows, int group, int64_t ld, float eps) {
  switch (io_dtype) {
    case GDN_DTYPE_BF16: launch_norm<D, GDN_DTYPE_BF16>(grid, st, x, gate, w, w_dtype, out, rows, group, ld, eps); break;
    case GDN_DTYPE_F16: launch_norm<D, GDN_DTYPE_F16>(grid, st, x, gate, w, w_dtype, out, rows, group, ld, eps); break;
    default: launch_norm<D, GDN_DTYPE_F32>(grid, st, x, gate, w, w_dtype, out, rows, group, ld, eps); break;
  }
}

}  // namespace

extern "C" int gdn_gated_rmsnorm(const void* x, const void* gate, int io_dtype, int64_t gate_group,
                                 int64_t gate_stride, const void* weight, int w_dtype, void* out, int64_t rows,
                                 int64_t D, float eps, void* stream) {
  using gdn_host::fail;
  if (rows < 0) return fail(GDN_ERR_INVALID, "gdn_gated_rmsnorm: rows must be >= 0");
  if (D != 64 && D != 128 && D != 256)
    return fail(GDN_ERR_UNSUPPORTED, "gdn_gated_rmsnorm: D must be 64, 128 or 256 (got %lld)", (long long)D);
  if (!gdn_host::dtype_ok(io_dtype) || !gdn_host::dtype_ok(w_dtype))
    return fail(GDN_ERR_INVALID, "gdn_gated_rmsnorm: bad dtype code");
  if (!(eps >= 0.0f)) return fail(GDN_ERR_INVALID, "gdn_gated_rmsnorm: eps must be >= 0");
  if (rows > 0 && (x == nullptr || gate == nullptr || out == nullptr))
    return fail(GDN_ERR_INVALID, "gdn_gated_rmsnorm: x, gate and out are required");
  if (!gdn_host::aligned(x, 16) || !gdn_host::aligned(gate, 16) || !gdn_host::aligned(out, 16) ||
      !gdn_host::aligned(weight, 16))
    return fail(GDN_ERR_INVALID, "gdn_gated_rmsnorm: pointers must be 16-byte aligned");
  if (gate_group < 0 || gate_stride < 0 || (gate_group > 0 && gate_stride < gate_group * D) || gate_group > INT32_MAX ||
      (gate_stride * (io_dtype == GDN_DTYPE_F32 ? 4 : 2)) % 16 != 0)
    return fail(GDN_ERR_INVALID, "gdn_gated_rmsnorm: gate lines of %lld rows, %lld apart, are not a valid layout",
                (long long)gate_group, (long long)gate_stride);
  if (rows == 0) return GDN_OK;
  // contiguous gate: one line of all rows
  const int group = gate_group > 0 ? static_cast<int>(gate_group) : 1;
  const int64_t ld = gate_group > 0 ? gate_stride : D;
  const int64_t rpb = kThreads / (D / CPL);
  const int64_t blocks = (rows + rpb - 1) / rpb;
  if (blocks > INT32_MAX || rows > INT32_MAX)
    return fail(GDN_ERR_UNSUPPORTED, "gdn_gated_rmsnorm: too many rows");
  const dim3 grid(static_cast<unsigned>(blocks));
  hipStream_t st = static_cast<hipStream_t>(stream);
  switch (D) {
    case 64: launch_norm_dt<64>(io_dtype, grid, st, x, gate, weight, w_dtype, out, rows, group, ld, eps); break;
    case 128: launch_norm_dt<128>(io_dtype, grid, st, x, gate, weight, w_dtype, out, rows, group, ld, eps); break;
    default: launch_norm_dt<256>(io_dtype, grid, st, x, gate, weight, w_dtype, out, rows, group, ld, eps); break;
  }
  return gdn_host::check_launch("gdn_gated_rmsnorm");
}
