// Fused GatedDeltaNet prologue: depthwise causal conv1d (4 taps) + SiLU +
// q/k RMS-norm + scales + conv-state update, and the conv-state commit of a
// partially accepted verify.  Bound by HBM: each mixed-qkv element is read
// once and each q/k/v element written once.
//
// A lane owns 8 adjacent channels (one 16-byte access of a bf16 row), so a
// head of D channels spans D/8 lanes and a wavefront covers 512/D heads.  A
// wavefront walks a run of consecutive tokens with a sliding window of the
// previous 3 inputs in registers, so the causal conv needs no re-reads; the
// per-token q/k norm is a DPP reduction over the head's lanes.
#include "gdn_common.hpp"

namespace {

using namespace gdn;

// Tokens per wavefront (prefill).  8 keeps the kernel at four waves per SIMD
// (109 VGPRs with the conv in fp32 FMAs, 88 on bf16 pairs; 16 tokens took
// 142, three waves), and re-reads the 3-row window once per 8 tokens (from
// L2).
constexpr int kRun = 8;
constexpr int kWaves = 4;  // wavefronts per workgroup (consecutive runs)
constexpr int KT = 4;      // conv taps

struct ProParams {
  const void* qkv;
  const void* cs_in;
  const void* weight;
  int w_dtype;
  const uint8_t* mask;
  const int32_t* cu_seqlens;
  void* q_out;
  void* k_out;
  void* v_out;
  void* cs_out;
  int n_seqs, S, Hk, Hv, C;
  int64_t ld;  // elements from one qkv row to the next (>= C)
  float eps;
};

// Locates (sequence, first token, length, run) of this workgroup.  Packed
// mode: sequence n owns max(1, ceil(len / RW)) run slots (one even when
// empty: its wave passes the conv state through), from cu[n] / RW + n on.
// With cu[n] = a RW + r, those end at or below floor(cu[n+1] / RW) + n + 1,
// the next sequence's first slot, and all lie below n_tok / RW + n_seqs (the
// grid); a workgroup finds its sequence by bisection.
template <int R>
__device__ __forceinline__ bool locate(const ProParams& p, int& seq, int64_t& start, int& len,
                                       int& run) {
  constexpr int RW = R * kWaves;
  run = blockIdx.y;
  if (p.cu_seqlens == nullptr) {
    seq = blockIdx.z;
    start = static_cast<int64_t>(seq) * p.S;
    len = p.S;
    return true;
  }
  // Offsets from a device tensor are not validated on the host: each
  // sequence is clamped into [0, S] (S = the packed token count), so a bad
  // table gives wrong rows but every run slot and token stays in bounds.
  auto cu_start = [&](int n) { return min(max(p.cu_seqlens[n], 0), p.S); };
  auto first_run = [&](int n) { return cu_start(n) / RW + n; };
  int lo = 0, hi = p.n_seqs - 1;  // the last sequence whose first slot is at or below run
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (first_run(mid) <= run) lo = mid;
    else hi = mid - 1;
  }
  const int s0 = cu_start(lo);
  const int l = min(max(p.cu_seqlens[lo + 1], s0), p.S) - s0;
  const int i = run - first_run(lo);
  if (i < 0 || i >= (l > 0 ? (l + RW - 1) / RW : 1)) return false;  // a slot no sequence uses
  seq = lo;
  start = s0;
  len = l;
  run = i;
  return true;
}

// W32: conv taps are fp32 (else they share the io dtype DT).  MASK: a token
// mask is given (without one no mask bytes are read or applied).  R: tokens
// per wavefront (16 for prefill; 1 and 4 for decode and verify rows, so a
// short row does not compute a 16-token run).
template <int D, int DT, bool W32, bool MASK, int R>
__global__ __launch_bounds__(256) void prologue_kernel(const ProParams p) {
  constexpr int LPH = D / CPL;   // lanes per head
  constexpr int HPW = 64 / LPH;  // heads per wavefront
  constexpr int WDT = W32 ? GDN_DTYPE_F32 : DT;
  constexpr bool kPairs = DT == GDN_DTYPE_BF16 && !W32;  // the conv on bf16 pairs (conv_pairs)
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform
  int seq, len, run;
  int64_t start;
  if (!locate<R>(p, seq, start, len, run)) return;
  const int t_begin = run * (R * kWaves) + wave * R;
  if (t_begin >= len && !(len == 0 && t_begin == 0)) return;
  const int t_end = t_begin + R < len ? t_begin + R : len;

  // This lane's head (over the 2 Hk + Hv heads of the mixed row) and its 8
  // channels; lanes past the last head work on a copy of it and store nothing.
  const int n_heads = 2 * p.Hk + p.Hv;
  const int head_all = blockIdx.x * HPW + lane / LPH;
  const bool active = head_all < n_heads;
  const int hg = active ? head_all : n_heads - 1;
  const int c0 = hg * D + (lane % LPH) * CPL;
  const int64_t C = p.C;

  // X = concat(conv_state (KT-1 rows), masked qkv): row xi of it (a masked
  // row is zeros).
  auto load_x = [&](int xi, float (&dst)[CPL]) {
    if (xi < KT - 1) {
      if (p.cs_in != nullptr) {
        unpack8<DT>(load_raw8<DT>(p.cs_in, (static_cast<int64_t>(seq) * (KT - 1) + xi) * C + c0), dst);
      } else {
#pragma unroll
        for (int j = 0; j < CPL; ++j) dst[j] = 0.0f;
      }
    } else {
      const int64_t tok = start + xi - (KT - 1);
      unpack8<DT>(load_raw8<DT>(p.qkv, tok * p.ld + c0), dst);
      if constexpr (MASK) {
        const bool keep = p.mask[tok] != 0;
#pragma unroll
        for (int j = 0; j < CPL; ++j) dst[j] = keep ? dst[j] : 0.0f;
      }
    }
  };
  if (t_end == t_begin) {
    // empty sequence: the conv state passes through
    if (p.cs_out != nullptr && active) {
#pragma unroll
      for (int i = 0; i < KT - 1; ++i) {
        float r[CPL];
        load_x(i, r);
        store8<DT>(p.cs_out, (static_cast<int64_t>(seq) * (KT - 1) + i) * C + c0, r);
      }
    }
    return;
  }
  // Issue every load first, in the order they are needed (memory returns in
  // issue order, so a wait for the taps or the window would otherwise also
  // wait for every token row queued ahead of them): the taps, the window of
  // the 3 inputs before the run, then the run's tokens (rows past the end
  // re-read the last row and are never stored).  All are raw loads, unpacked
  // only once every load is issued, so token u is computed as soon as its
  // own row arrives.  A masked token reads as zero: a select, as the
  // reference's where(mask, qkv, 0), so a non-finite value in a masked row
  // reaches no output.
  Raw8<WDT> wr[KT];  // taps of the lane's 8 channels: weight[c][tap], 32 consecutive values
#pragma unroll
  for (int i = 0; i < KT; ++i) wr[i] = load_raw8<WDT>(p.weight, static_cast<int64_t>(c0) * KT + 8 * i);
  // window row i = X[t + i] for the run's first token t: a conv-state row
  // for t + i < KT - 1, else a qkv row.  Without a conv state those rows are
  // zeros: the sequence's first qkv row is read and then zeroed (wm = 0),
  // so the load stays unconditional and in the global address space.
  Raw8<DT> xw[KT - 1];
  float wm[KT - 1];
#pragma unroll
  for (int i = 0; i < KT - 1; ++i) {
    const int xi = t_begin + i;
    const bool from_cs = xi < KT - 1;
    const bool cs_row = from_cs && p.cs_in != nullptr;
    const int64_t tok = from_cs ? start : start + xi - (KT - 1);
    const int64_t off = cs_row ? (static_cast<int64_t>(seq) * (KT - 1) + xi) * C + c0 : tok * p.ld + c0;
    xw[i] = load_raw8<DT>(cs_row ? p.cs_in : p.qkv, off);
    wm[i] = from_cs ? (cs_row ? 1.0f : 0.0f) : 1.0f;
    if constexpr (MASK) {
      if (!from_cs) wm[i] = p.mask[tok] != 0 ? 1.0f : 0.0f;
    }
  }
  Raw8<DT> xs[R];
  float xm[R];
  const int t_last = t_end - 1;
#pragma unroll
  for (int u = 0; u < R; ++u) {
    const int64_t tok = start + min(t_begin + u, t_last);
    xs[u] = load_raw8<DT>(p.qkv, tok * p.ld + c0);
    if constexpr (MASK) xm[u] = p.mask[tok] != 0 ? 1.0f : 0.0f;
  }
  // Head role: 0 = q, 1 = k, 2 = v (lanes of one head agree).
  const int role = hg < p.Hk ? 0 : (hg < 2 * p.Hk ? 1 : 2);
  const int head = role == 0 ? hg : (role == 1 ? hg - p.Hk : hg - 2 * p.Hk);
  void* out = role == 0 ? p.q_out : (role == 1 ? p.k_out : p.v_out);
  const int H = role == 2 ? p.Hv : p.Hk;
  const float post = role == 0 ? 1.0f / static_cast<float>(D) : rsqrtf(static_cast<float>(D));
  // output row of the run's first token; one row = H * D elements
  constexpr int ES = DT == GDN_DTYPE_F32 ? 4 : 2;
  char* orow = static_cast<char*>(out) + ((start + t_begin) * H * D + static_cast<int64_t>(head) * D +
                                          (lane % LPH) * CPL) * ES;
  const int64_t ostep = static_cast<int64_t>(H) * D * ES;
  const int64_t cs_row0 = static_cast<int64_t>(seq) * (KT - 1) * C + c0;  // the lane's slice of conv-state row 0

  // Token u's SiLU outputs o (and their sum of squares): the q/k norm over
  // the head's lanes (every lane takes part in the DPP reduction; v heads
  // keep scale 1), then the store of a real token.
  auto finish = [&](int u, float (&o)[CPL], float ss) {
    ss = head_sum<LPH>(ss);
    const float sc = role == 2 ? 1.0f : rsqrtf(ss / static_cast<float>(D) + p.eps) * post;
#pragma unroll
    for (int j = 0; j < CPL; ++j) o[j] *= sc;
    if (active && t_begin + u < t_end) store8<DT>(orow, 0, o);
    orow += ostep;
  };
  // The new conv state is the last KT-1 rows of X (the wave holding the
  // sequence's last token writes it).  With one-token runs the window has
  // just shifted onto exactly those rows (masked, as load_x reads them);
  // longer runs have run past them and read them again.
  const bool write_cs = t_end == len && p.cs_out != nullptr && active;

  // Every token of the run is computed (tokens past the end repeat the last
  // row, so no control flow splits the window); only real tokens are stored.
  if constexpr (kPairs) {
    // bf16 rows and taps: the conv on bf16 pairs (conv_pairs), with the
    // taps as loaded and absent or masked rows as zeros
    uint32_t w01[CPL], w23[CPL];
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
      w01[j] = wr[j >> 1].v[2 * (j & 1)];
      w23[j] = wr[j >> 1].v[2 * (j & 1) + 1];
    }
    u32x4 rw[KT - 1];  // X_{t-3}, X_{t-2}, X_{t-1} of the current token t
#pragma unroll
    for (int i = 0; i < KT - 1; ++i) rw[i] = row_or_zero(wm[i] != 0.0f, xw[i].v);
    uint32_t pa[CPL], pb[CPL];  // p(t - 2), p(t - 1)
    row_pairs(rw[0], rw[1], pa);
    row_pairs(rw[1], rw[2], pb);
#pragma unroll
    for (int u = 0; u < R; ++u) {
      u32x4 xr = xs[u].v;
      if constexpr (MASK) xr = row_or_zero(xm[u] != 0.0f, xr);
      uint32_t pc[CPL];  // p(t)
      row_pairs(rw[KT - 2], xr, pc);
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
      rw[0] = rw[1];
      rw[1] = rw[2];
      rw[2] = xr;
      finish(u, o, ss);
    }
    if (write_cs) {
#pragma unroll
      for (int i = 0; i < KT - 1; ++i) {
        if constexpr (R == 1) {
          *reinterpret_cast<u32x4*>(static_cast<uint16_t*>(p.cs_out) + cs_row0 + i * C) = rw[i];
        } else {
          float r[CPL];
          load_x(len + i, r);
          store8<DT>(p.cs_out, cs_row0 + i * C, r);
        }
      }
    }
  } else {
    float w[KT][CPL];
    {
      float wv[CPL * KT];
#pragma unroll
      for (int i = 0; i < KT; ++i) unpack8<WDT>(wr[i], *reinterpret_cast<float(*)[CPL]>(&wv[8 * i]));
#pragma unroll
      for (int j = 0; j < CPL; ++j)
#pragma unroll
        for (int i = 0; i < KT; ++i) w[i][j] = wv[j * KT + i];
    }
    float win[KT - 1][CPL];
#pragma unroll
    for (int i = 0; i < KT - 1; ++i) {
      unpack8<DT>(xw[i], win[i]);
#pragma unroll
      for (int j = 0; j < CPL; ++j) win[i][j] = wm[i] != 0.0f ? win[i][j] : 0.0f;
    }
#pragma unroll
    for (int u = 0; u < R; ++u) {
      float x[CPL], o[CPL];
      unpack8<DT>(xs[u], x);
      float ss = 0.0f;
#pragma unroll
      for (int j = 0; j < CPL; ++j) {
        if constexpr (MASK) x[j] = xm[u] != 0.0f ? x[j] : 0.0f;
        float acc = w[KT - 1][j] * x[j];
#pragma unroll
        for (int i = 0; i < KT - 1; ++i) acc = fmaf(w[i][j], win[i][j], acc);
        o[j] = silu(acc);
        ss = fmaf(o[j], o[j], ss);
      }
#pragma unroll
      for (int i = 0; i < KT - 2; ++i)
#pragma unroll
        for (int j = 0; j < CPL; ++j) win[i][j] = win[i + 1][j];
#pragma unroll
      for (int j = 0; j < CPL; ++j) win[KT - 2][j] = x[j];
      finish(u, o, ss);
    }
    if (write_cs) {
#pragma unroll
      for (int i = 0; i < KT - 1; ++i) {
        float r[CPL];
        if constexpr (R == 1) {
#pragma unroll
          for (int j = 0; j < CPL; ++j) r[j] = win[i][j];
        } else {
          load_x(len + i, r);
        }
        store8<DT>(p.cs_out, cs_row0 + i * C, r);
      }
    }
  }
}

template <int DT>
__global__ __launch_bounds__(256) void conv_commit_kernel(const void* cs_in, const void* qkv,
                                                          const uint8_t* mask,
                                                          const int32_t* n_commit, void* cs_out,
                                                          int T, int C, int64_t ld, int KT1, int64_t total) {
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (idx >= total) return;
  const int c = static_cast<int>(idx % C);
  const int64_t bi = idx / C;
  const int i = static_cast<int>(bi % KT1);
  const int64_t b = bi / KT1;
  int n = n_commit[b];
  n = n < 0 ? 0 : (n > T ? T : n);
  const int xi = n + i;  // row of concat(conv_state, qkv)
  float val;
  if (xi < KT1) {
    val = cs_in != nullptr ? IO<DT>::load1(cs_in, (b * KT1 + xi) * C + c) : 0.0f;
  } else {
    const int64_t tok = b * T + (xi - KT1);
    val = (mask == nullptr || mask[tok] != 0) ? IO<DT>::load1(qkv, tok * ld + c) : 0.0f;
  }
  IO<DT>::store1(cs_out, idx, val);
}

}  // namespace

extern "C" int gdn_conv_prologue(const void* qkv, int io_dtype, int64_t qkv_stride, const void* conv_state_in,
                                 const void* weight, int w_dtype, const uint8_t* mask,
                                 const int32_t* cu_seqlens, void* q_out, void* k_out,
                                 void* v_out, void* conv_state_out, int64_t B, int64_t S,
                                 int64_t Hk, int64_t Hv, int64_t Dk, int64_t Dv, int64_t Kt,
                                 float eps, void* stream) {
  using gdn_host::fail;
  if (B < 0 || S < 0 || Hk <= 0 || Hv <= 0)
    return fail(GDN_ERR_INVALID, "gdn_conv_prologue: bad sizes");
  if (Dk != Dv || (Dk != 64 && Dk != 128 && Dk != 256))
    return fail(GDN_ERR_UNSUPPORTED, "gdn_conv_prologue: needs Dk == Dv in {64,128,256} (got %lld, %lld)",
                (long long)Dk, (long long)Dv);
  if (Kt != KT) return fail(GDN_ERR_UNSUPPORTED, "gdn_conv_prologue: only Kt=4 is built (got %lld)", (long long)Kt);
  if (!gdn_host::dtype_ok(io_dtype) || !gdn_host::dtype_ok(w_dtype))
    return fail(GDN_ERR_INVALID, "gdn_conv_prologue: bad dtype code");
  if (w_dtype != io_dtype && w_dtype != GDN_DTYPE_F32)
    return fail(GDN_ERR_UNSUPPORTED, "gdn_conv_prologue: conv weight must be fp32 or the qkv dtype");
  if (qkv == nullptr || weight == nullptr || q_out == nullptr || k_out == nullptr || v_out == nullptr)
    return fail(GDN_ERR_INVALID, "gdn_conv_prologue: qkv, weight and q/k/v outputs are required");
  // In place only for unpacked rows of at most one token: one wave then reads
  // each row's whole window (its registers hold it) before it writes the
  // row's new state, and no other wave touches that row.
  if (conv_state_out != nullptr && conv_state_out == conv_state_in && (cu_seqlens != nullptr || S > 1))
    return fail(GDN_ERR_INVALID,
                "gdn_conv_prologue: conv_state_out may alias conv_state_in only for unpacked rows of one token");
  if (!(eps >= 0.0f)) return fail(GDN_ERR_INVALID, "gdn_conv_prologue: eps must be >= 0");
  if (qkv_stride != 0 && (qkv_stride < 2 * Hk * Dk + Hv * Dv || (qkv_stride * (io_dtype == GDN_DTYPE_F32 ? 4 : 2)) % 16 != 0))
    return fail(GDN_ERR_INVALID, "gdn_conv_prologue: qkv_stride=%lld must be >= C and keep rows 16-byte aligned",
                (long long)qkv_stride);
  if (!gdn_host::aligned(qkv, 16) || !gdn_host::aligned(q_out, 16) || !gdn_host::aligned(k_out, 16) ||
      !gdn_host::aligned(v_out, 16) || !gdn_host::aligned(conv_state_in, 16) ||
      !gdn_host::aligned(conv_state_out, 16) || !gdn_host::aligned(weight, 16))
    return fail(GDN_ERR_INVALID, "gdn_conv_prologue: pointers must be 16-byte aligned");
  if (B == 0) return GDN_OK;
  if (B > 65535 || S > INT32_MAX / 2)
    return fail(GDN_ERR_UNSUPPORTED, "gdn_conv_prologue: B or S too large");

  ProParams p;
  p.qkv = qkv;
  p.cs_in = conv_state_in;
  p.weight = weight;
  p.w_dtype = w_dtype;
  p.mask = mask;
  p.cu_seqlens = cu_seqlens;
  p.q_out = q_out;
  p.k_out = k_out;
  p.v_out = v_out;
  p.cs_out = conv_state_out;
  p.n_seqs = static_cast<int>(B);
  p.S = static_cast<int>(S);
  p.Hk = static_cast<int>(Hk);
  p.Hv = static_cast<int>(Hv);
  p.C = static_cast<int>(2 * Hk * Dk + Hv * Dv);
  p.ld = qkv_stride > 0 ? qkv_stride : p.C;
  p.eps = eps;

  // tokens per wavefront: short unpacked rows (decode, verify) take a short run
  const int run = (cu_seqlens == nullptr && S <= 1) ? 1 : ((cu_seqlens == nullptr && S <= 4) ? 4 : kRun);
  const int64_t RW = static_cast<int64_t>(run) * kWaves;
  dim3 block(64 * kWaves);
  dim3 grid;
  const int64_t heads_per_wave = 512 / Dk;  // a lane covers 8 channels
  grid.x = static_cast<unsigned>((2 * Hk + Hv + heads_per_wave - 1) / heads_per_wave);
  if (cu_seqlens != nullptr) {
    grid.y = static_cast<unsigned>((S + RW - 1) / RW + B);
    grid.z = 1;
  } else {
    grid.y = static_cast<unsigned>(S > 0 ? (S + RW - 1) / RW : 1);
    grid.z = static_cast<unsigned>(B);
  }
  hipStream_t st = static_cast<hipStream_t>(stream);
#define GDN_PRO_LAUNCH_R(D_, DT_, W_, M_)                                                   \
  if (run == 1)                                                                            \
    hipLaunchKernelGGL((prologue_kernel<D_, DT_, W_, M_, 1>), grid, block, 0, st, p);      \
  else if (run == 4)                                                                       \
    hipLaunchKernelGGL((prologue_kernel<D_, DT_, W_, M_, 4>), grid, block, 0, st, p);      \
  else                                                                                     \
    hipLaunchKernelGGL((prologue_kernel<D_, DT_, W_, M_, kRun>), grid, block, 0, st, p)
#define GDN_PRO_LAUNCH_M(D_, DT_, W_)    \
  if (mask != nullptr) {                 \
    GDN_PRO_LAUNCH_R(D_, DT_, W_, true);  \
  } else {                               \
    GDN_PRO_LAUNCH_R(D_, DT_, W_, false); \
  }
#define GDN_PRO_LAUNCH(D_, DT_)            \
  if (w_dtype == GDN_DTYPE_F32) {          \
    GDN_PRO_LAUNCH_M(D_, DT_, true);       \
  } else {                                 \
    GDN_PRO_LAUNCH_M(D_, DT_, false);      \
  }
#define GDN_PRO_DT(D_)                                             \
  switch (io_dtype) {                                             \
    case GDN_DTYPE_BF16: GDN_PRO_LAUNCH(D_, GDN_DTYPE_BF16); break; \
    case GDN_DTYPE_F16: GDN_PRO_LAUNCH(D_, GDN_DTYPE_F16); break;   \
    default: GDN_PRO_LAUNCH(D_, GDN_DTYPE_F32); break;              \
  }
  switch (Dk) {
    case 64: GDN_PRO_DT(64); break;
    case 128: GDN_PRO_DT(128); break;
    default: GDN_PRO_DT(256); break;
  }
#undef GDN_PRO_DT
#undef GDN_PRO_LAUNCH
#undef GDN_PRO_LAUNCH_M
#undef GDN_PRO_LAUNCH_R
  return gdn_host::check_launch("gdn_conv_prologue");
}

extern "C" int gdn_conv_state_commit(const void* conv_state_in, const void* qkv, int io_dtype,
                                     int64_t qkv_stride, const uint8_t* mask, const int32_t* n_commit,
                                     void* conv_state_out, int64_t B, int64_t T, int64_t C,
                                     int64_t Kt, void* stream) {
  using gdn_host::fail;
  if (B < 0 || T < 0 || C <= 0 || Kt < 2)
    return fail(GDN_ERR_INVALID, "gdn_conv_state_commit: bad sizes");
  if (!gdn_host::dtype_ok(io_dtype)) return fail(GDN_ERR_INVALID, "gdn_conv_state_commit: bad dtype");
  if (qkv == nullptr || n_commit == nullptr || conv_state_out == nullptr)
    return fail(GDN_ERR_INVALID, "gdn_conv_state_commit: qkv, n_commit and conv_state_out are required");
  if (conv_state_out == conv_state_in)
    return fail(GDN_ERR_INVALID, "gdn_conv_state_commit: conv_state_out must not alias conv_state_in");
  if (qkv_stride != 0 && qkv_stride < C)
    return fail(GDN_ERR_INVALID, "gdn_conv_state_commit: qkv_stride=%lld is below C=%lld", (long long)qkv_stride,
                (long long)C);
  const int64_t ld = qkv_stride > 0 ? qkv_stride : C;
  const int64_t total = B * (Kt - 1) * C;
  if (total == 0) return GDN_OK;
  if (T > INT32_MAX || C > INT32_MAX) return fail(GDN_ERR_UNSUPPORTED, "gdn_conv_state_commit: too large");
  const int threads = 256;
  const int64_t blocks = (total + threads - 1) / threads;
  if (blocks > INT32_MAX) return fail(GDN_ERR_UNSUPPORTED, "gdn_conv_state_commit: too large");
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int Ti = static_cast<int>(T), Ci = static_cast<int>(C), K1 = static_cast<int>(Kt - 1);
  switch (io_dtype) {
    case GDN_DTYPE_BF16:
      hipLaunchKernelGGL((conv_commit_kernel<GDN_DTYPE_BF16>), dim3(blocks), dim3(threads), 0, st,
                         conv_state_in, qkv, mask, n_commit, conv_state_out, Ti, Ci, ld, K1, total);
      break;
    case GDN_DTYPE_F16:
      hipLaunchKernelGGL((conv_commit_kernel<GDN_DTYPE_F16>), dim3(blocks), dim3(threads), 0, st,
                         conv_state_in, qkv, mask, n_commit, conv_state_out, Ti, Ci, ld, K1, total);
      break;
    default:
      hipLaunchKernelGGL((conv_commit_kernel<GDN_DTYPE_F32>), dim3(blocks), dim3(threads), 0, st,
                         conv_state_in, qkv, mask, n_commit, conv_state_out, Ti, Ci, ld, K1, total);
      break;
  }
  return gdn_host::check_launch("gdn_conv_state_commit");
}
