/*
 * gdn.h -- C ABI of libgdn.so, the MI355X (gfx950) Gated DeltaNet hot path.
 *
 * Every entry point takes plain device pointers and sizes, enqueues work on
 * the given HIP stream (a hipStream_t passed as void*, NULL = default
 * stream) and returns immediately.  Nothing here allocates device memory or
 * synchronises: the caller owns every buffer, including workspaces, and the
 * pointers are borrowed only for the enqueue.
 *
 * Return value: GDN_OK (0) or a negative status.  Argument errors are
 * detected before any HIP call, so they are reported identically with or
 * without a GPU.  gdn_last_error() gives a message for the calling thread.
 *
 * Layouts (row-major, contiguous, batch-major with heads before head dim,
 * as mlx-lm lays them out):
 *   q, k   [B, T, Hk, Dk]          v, y   [B, T, Hv, Dv]
 *   a, b, g, beta  [B, T, Hv]      A_log, dt_bias  [Hv]
 *   state  [B, Hv, Dv, Dk] fp32 (Dk innermost)     mask  [B, T] uint8 (0/1)
 * Packed ragged sequences (cu_seqlens != NULL): B is the number of
 * sequences, tensors are [1, N_tok, ...] and sequence n owns tokens
 * [cu_seqlens[n], cu_seqlens[n+1]); state rows are per sequence.
 * GQA: v-head h reads q/k head h / (Hv / Hk).
 *
 * Recurrence per (sequence, v-head), S in R^{Dv x Dk}:
 *   g = exp(-exp(A_log) * softplus(a + dt_bias)),  beta = sigmoid(b)
 *   S <- g S;  kv = S k;  S <- S + beta (v - kv) k^T;  y = S q
 * A token whose mask byte is 0 leaves S unchanged and gets y = 0.
 */
#ifndef GDN_H
#define GDN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define GDN_ABI_VERSION 4

/* dtype codes for the void* operands */
#define GDN_DTYPE_F32 0
#define GDN_DTYPE_BF16 1
#define GDN_DTYPE_F16 2

/* gate modes of gdn_recurrent_args.gate_mode / gdn_chunk_fwd */
#define GDN_GATES_RAW 0 /* gx = a, gy = b, with A_log and dt_bias   */
#define GDN_GATES_PRE 1 /* gx = g, gy = beta (already transformed)  */

/* status codes */
#define GDN_OK 0
#define GDN_ERR_LAUNCH (-5)       /* a HIP call failed               */
#define GDN_ERR_INVALID (-22)     /* bad pointer / shape / dtype      */
#define GDN_ERR_UNSUPPORTED (-95) /* valid but not built (e.g. Dk)    */

/* Version of this ABI (GDN_ABI_VERSION of the built library). */
int gdn_abi_version(void);

/* Message for the last failing call on this thread ("" if none). */
const char* gdn_last_error(void);

/*
 * mlx-lm gated_delta_update(q, k, v, a, b, A_log, dt_bias, state, mask):
 * replaces the fused entry point multiplex calls at
 * multiplex/kernel/dflash.py:372-374 and :417-422 (reached from
 * multiplex/kernel/engine.py:164-167).  The gate transforms are fused.
 * state_in NULL = zero state; mask NULL = all tokens active.  y and
 * state_out are written (state_out may alias state_in for in-place use).
 */
int gdn_gated_delta_update(const void* q, const void* k, const void* v, int qkv_dtype,
                           const void* a, const void* b, int ab_dtype,
                           const void* A_log, const void* dt_bias, int param_dtype,
                           const float* state_in, const uint8_t* mask,
                           void* y, float* state_out,
                           int64_t B, int64_t T, int64_t Hk, int64_t Hv,
                           int64_t Dk, int64_t Dv, void* stream);

/*
 * mlx-lm gated_delta_kernel(q, k, v, g, beta, state, mask): the same
 * recurrence with the decay g and write strength beta precomputed
 * (mlx-lm dispatches to it from gated_delta_update, dflash.py:373).
 */
int gdn_gated_delta_kernel(const void* q, const void* k, const void* v, int qkv_dtype,
                           const void* g, const void* beta, int gb_dtype,
                           const float* state_in, const uint8_t* mask,
                           void* y, float* state_out,
                           int64_t B, int64_t T, int64_t Hk, int64_t Hv,
                           int64_t Dk, int64_t Dv, void* stream);

/*
 * General recurrent launch (decode, MTP verify, commit, ragged rows).
 * Replaces the verify forward plus the replay rollback of
 * multiplex/kernel/engine.py:337-359 and dflash.py:403-426.
 *   state_out  NULL: the state is not written (verify without commit).
 *   snapshots  [B,T,Hv,Dv,Dk] fp32 (or [N_tok,...] packed): the state after
 *              every token (for rollback by index), NULL = none.
 *   y          NULL: outputs not computed (commit-only launch).
 *   commit_len [B] int32: row b writes the state after its first
 *              commit_len[b] tokens (0 = initial state, < 0 = no write,
 *              > length = clamped); NULL = after all tokens.
 *   state_index [B] int32 or NULL: pooled states.  state_in and state_out
 *              are then pools of n_slots states [n_slots,Hv,Dv,Dk], and row
 *              b reads and writes slot state_index[b] (state_in NULL = a
 *              zero initial state; state_out == state_in updates the pool
 *              in place).  Batch membership changes (join, leave, filter,
 *              merge of the scheduler, engine.py:383-432) then move int32
 *              indices, not 2 MiB states.  A row whose index is outside
 *              [0, n_slots) is not processed: its y and its slot are left
 *              as they are.  Rows that write state must use distinct slots.
 *              No counterpart in the reference, which concatenates states.
 *   gate_stride elements from one token's gate row (gx, gy) to the next,
 *              >= Hv; 0 = Hv (contiguous).  Lets a and b be column slices of
 *              one fused in_proj output.
 * Rows run independently; a launch never reads another row's state.
 */
typedef struct gdn_recurrent_args {
  const void* q;
  const void* k;
  const void* v;
  int32_t qkv_dtype;
  int32_t gate_mode;   /* GDN_GATES_RAW / GDN_GATES_PRE */
  const void* gx;      /* a or g      [B,T,Hv] */
  const void* gy;      /* b or beta   [B,T,Hv] */
  int32_t gate_dtype;
  int32_t param_dtype; /* A_log / dt_bias (raw mode only) */
  const void* A_log;
  const void* dt_bias;
  const float* state_in;
  float* state_out;
  float* snapshots;
  void* y;
  const uint8_t* mask;
  const int32_t* cu_seqlens; /* [B+1] or NULL */
  const int32_t* commit_len; /* [B] or NULL */
  const int32_t* state_index; /* [B] or NULL: slots of pooled states */
  int64_t B, T;              /* T = tokens per row, or N_tok when packed */
  int64_t Hk, Hv, Dk, Dv;
  int64_t n_slots;           /* pool size when state_index != NULL */
  int64_t gate_stride;       /* elements between tokens' gate rows (0 = Hv) */
  void* stream;
  int64_t y_from;            /* tokens before it produce no y (not written); 0 = all */
} gdn_recurrent_args;

int gdn_recurrent(const gdn_recurrent_args* args);

/*
 * Chunked (WY/UT) prefill of packed ragged sequences on bf16 MFMA; the
 * long-T form of gdn_gated_delta_update (the reference runs prefill chunks
 * of 512 tokens through the sequential kernel, multiplex/kernel/
 * scheduler.py:331-333 -> engine.py:261-269).  q/k/v must be bf16.
 * cu_seqlens [n_seqs+1] (NULL: n_seqs rows of n_tok/n_seqs tokens each,
 * [B,T,...] layout).  state_in [n_seqs,Hv,Dv,Dk] fp32 or NULL (zeros),
 * state_out may alias state_in.  state_index [n_seqs] int32 or NULL:
 * pooled states as in gdn_recurrent_args (state_in / state_out are pools of
 * n_slots states; sequence n uses slot state_index[n]; out-of-range slots
 * are skipped).  gate_stride as in gdn_recurrent_args.  mask [n_tok] uint8 or
 * NULL: a token whose byte is 0 keeps the state and its y is 0 (as in
 * gdn_recurrent).  chunk must be 64.
 * workspace must hold gdn_chunk_workspace_bytes(...) bytes (256-B aligned).
 */
size_t gdn_chunk_workspace_bytes(int64_t n_seqs, int64_t n_tok, int64_t Hv,
                                 int64_t Dk, int64_t Dv, int64_t chunk);

int gdn_chunk_fwd(const void* q, const void* k, const void* v, int qkv_dtype,
                  int gate_mode, const void* gx, const void* gy, int gate_dtype,
                  int64_t gate_stride,
                  const void* A_log, const void* dt_bias, int param_dtype,
                  const uint8_t* mask, const float* state_in, void* y, float* state_out,
                  const int32_t* state_index, int64_t n_slots,
                  const int32_t* cu_seqlens, int64_t n_seqs, int64_t n_tok,
                  int64_t Hk, int64_t Hv, int64_t Dk, int64_t Dv, int64_t chunk,
                  void* workspace, size_t workspace_bytes, void* stream);

/*
 * The two phases of gdn_chunk_fwd, enqueued separately (same arguments, same
 * checks): gdn_chunk_prep writes the per-chunk records into the workspace
 * (every chunk in parallel; reads q, k and the gates, not the state), and
 * gdn_chunk_scan runs the state chain over them and writes y and state_out.
 * A scan must follow the prep of the same arguments and workspace on the
 * caller's streams.  The split lets a serving step place HBM-bound work (the
 * decode / verify / commit launches of other rows) beside the scan, which
 * leaves HBM mostly idle, instead of beside the prep, which is itself bound
 * by HBM.  No reference counterpart beyond gdn_chunk_fwd's: only where the
 * caller places the two launches changes.
 */
int gdn_chunk_prep(const void* q, const void* k, const void* v, int qkv_dtype,
                   int gate_mode, const void* gx, const void* gy, int gate_dtype,
                   int64_t gate_stride,
                   const void* A_log, const void* dt_bias, int param_dtype,
                   const uint8_t* mask, const float* state_in, void* y, float* state_out,
                   const int32_t* state_index, int64_t n_slots,
                   const int32_t* cu_seqlens, int64_t n_seqs, int64_t n_tok,
                   int64_t Hk, int64_t Hv, int64_t Dk, int64_t Dv, int64_t chunk,
                   void* workspace, size_t workspace_bytes, void* stream);
int gdn_chunk_scan(const void* q, const void* k, const void* v, int qkv_dtype,
                   int gate_mode, const void* gx, const void* gy, int gate_dtype,
                   int64_t gate_stride,
                   const void* A_log, const void* dt_bias, int param_dtype,
                   const uint8_t* mask, const float* state_in, void* y, float* state_out,
                   const int32_t* state_index, int64_t n_slots,
                   const int32_t* cu_seqlens, int64_t n_seqs, int64_t n_tok,
                   int64_t Hk, int64_t Hv, int64_t Dk, int64_t Dv, int64_t chunk,
                   void* workspace, size_t workspace_bytes, void* stream);

/*
 * The mixer's prefill from its mixed projection: the conv prologue
 * (gdn_conv_prologue; dflash.py:351-370) fused into gdn_chunk_fwd's prep,
 * then the scan (dflash.py:372-374).  Replaces gdn_conv_prologue followed by
 * gdn_chunk_fwd: the prep forms its chunk's q and k (its k-head) and v (its
 * v-head) from the qkv rows with the prologue's arithmetic, so y, the state
 * and the new conv state are bit-identical to that pair's, and q and k are
 * never written (v goes to the workspace, for the scan).
 *   qkv [n_tok, C] bf16 rows (C = 2 Hk Dk + Hv Dv, q | k | v channels),
 *       qkv_stride elements apart (0: C; else >= C, a multiple of 8);
 *   conv_w [C][4] taps, bf16 or fp32 (conv_w_dtype);
 *   conv_state_in [n_seqs][3][C] bf16 or NULL (zeros); conv_state_out the
 *       same shape or NULL (not written), not aliasing conv_state_in;
 *   eps: the q/k norms' epsilon.
 * Gates, states, sequences and y as in gdn_chunk_fwd (no mask; Dk = Dv =
 * 128).  The workspace must hold gdn_chunk_conv_workspace_bytes(...) bytes
 * (256-B aligned): gdn_chunk_workspace_bytes(...), then n_tok Hv Dv bf16.
 */
size_t gdn_chunk_conv_workspace_bytes(int64_t n_seqs, int64_t n_tok, int64_t Hv,
                                      int64_t Dk, int64_t Dv, int64_t chunk);

int gdn_chunk_fwd_conv(const void* qkv, int64_t qkv_stride, const void* conv_w,
                       int conv_w_dtype, const void* conv_state_in,
                       void* conv_state_out, float eps, int gate_mode,
                       const void* gx, const void* gy, int gate_dtype,
                       int64_t gate_stride, const void* A_log,
                       const void* dt_bias, int param_dtype,
                       const float* state_in, void* y, float* state_out,
                       const int32_t* state_index, int64_t n_slots,
                       const int32_t* cu_seqlens, int64_t n_seqs, int64_t n_tok,
                       int64_t Hk, int64_t Hv, int64_t Dk, int64_t Dv,
                       int64_t chunk, void* workspace, size_t workspace_bytes,
                       void* stream);

/*
 * gdn_chunk_fwd without a workspace argument: the chunk records go to a
 * static device array of 64 MiB (67,108,864 bytes) inside the library,
 * one per GPU, held until the process ends.  No reference counterpart: it
 * is for callers that cannot allocate device memory (code under HIP graph
 * capture, serving loops that forbid allocation).  Calls whose
 * gdn_chunk_workspace_bytes(...) exceed 64 MiB return GDN_ERR_UNSUPPORTED
 * before any HIP call (at Hv = 32: one sequence of up to 1536 tokens, or
 * packed sequences with ceil(n_tok / 64) + n_seqs <= 25).  The array's
 * address on the current device (which must be the stream's) is taken on
 * the first call there.  Every call on one GPU shares the array: calls that
 * overlap on one GPU (on different streams) race.  Other arguments as in
 * gdn_chunk_fwd.
 */
int gdn_chunk_fwd_noalloc(const void* q, const void* k, const void* v, int qkv_dtype,
                          int gate_mode, const void* gx, const void* gy, int gate_dtype,
                          int64_t gate_stride,
                          const void* A_log, const void* dt_bias, int param_dtype,
                          const uint8_t* mask, const float* state_in, void* y,
                          float* state_out,
                          const int32_t* state_index, int64_t n_slots,
                          const int32_t* cu_seqlens, int64_t n_seqs, int64_t n_tok,
                          int64_t Hk, int64_t Hv, int64_t Dk, int64_t Dv, int64_t chunk,
                          void* stream);

/*
 * Fused mixer prologue of GatedDeltaNet (dflash.py:351-370): mask zeroing,
 * concat(conv_state, qkv), depthwise causal conv1d with Kt taps (no bias),
 * SiLU, split into q | k | v, q = rms_norm(q)/Dk, k = rms_norm(k)/sqrt(Dk)
 * (rms_norm(x) = x / sqrt(mean(x^2) + eps)), and the new conv state
 * (last Kt-1 rows of the concat).
 *   qkv            [B,S,C] with C = 2*Hk*Dk + Hv*Dv, io_dtype
 *   conv_state_in  [B,Kt-1,C] io_dtype or NULL (zeros)
 *   weight         [C,Kt] w_dtype (mlx-lm's [C,Kt,1] squeezed)
 *   mask           [B,S] uint8 or NULL
 *   q_out, k_out   [B,S,Hk,Dk];  v_out [B,S,Hv,Dv]   (io_dtype)
 *   conv_state_out [B,Kt-1,C] or NULL; may be conv_state_in (updated in
 *                  place) only for unpacked rows of S <= 1 token (decode)
 *   qkv_stride     elements from one qkv row (token) to the next, >= C and
 *                  16-byte aligned; 0 = C.  Lets qkv be a column slice of one
 *                  fused in_proj output.
 * cu_seqlens: packed sequences as in gdn_chunk_fwd (B = n_seqs, S = n_tok).
 * Requires Dk == Dv in {64, 128, 256}.
 */
int gdn_conv_prologue(const void* qkv, int io_dtype, int64_t qkv_stride, const void* conv_state_in,
                      const void* weight, int w_dtype, const uint8_t* mask,
                      const int32_t* cu_seqlens,
                      void* q_out, void* k_out, void* v_out, void* conv_state_out,
                      int64_t B, int64_t S, int64_t Hk, int64_t Hv, int64_t Dk,
                      int64_t Dv, int64_t Kt, float eps, void* stream);

/*
 * Conv-state commit of a partially accepted verify (dflash.py:424-425):
 * conv_state_out[b] = concat(conv_state_in[b], masked qkv[b])[n : n+Kt-1]
 * with n = n_commit[b] in [0, T].  conv_state_out must not alias
 * conv_state_in.  qkv_stride as in gdn_conv_prologue.
 */
int gdn_conv_state_commit(const void* conv_state_in, const void* qkv, int io_dtype,
                          int64_t qkv_stride, const uint8_t* mask, const int32_t* n_commit,
                          void* conv_state_out, int64_t B, int64_t T, int64_t C,
                          int64_t Kt, void* stream);

/*
 * Gated RMSNorm of the mixer epilogue, self_layer.norm(out, z) at
 * dflash.py:377 (mlx-lm's gated norm; restated by transformers'
 * Qwen3NextRMSNormGated, models/qwen3_next/modeling_qwen3_next.py:57-74).
 * Per row of D channels:
 *   n = x / sqrt(mean(x^2) + eps)       rounded to io_dtype
 *   m = weight * n                      rounded to io_dtype if w_dtype == io_dtype
 *   out = m * silu(gate)                (fp32 product, rounded once)
 *   x, out  [rows, D] io_dtype;  weight [D] w_dtype, or NULL for ones
 *   gate     io_dtype: row r at (r / gate_group) * gate_stride +
 *            (r % gate_group) * D (lines of gate_group rows, e.g. one
 *            token's heads, gate_stride elements apart); gate_group = 0
 *            means [rows, D] contiguous.
 * out may alias x (or a contiguous gate).  Requires D in {64, 128, 256}.
 */
int gdn_gated_rmsnorm(const void* x, const void* gate, int io_dtype,
                      int64_t gate_group, int64_t gate_stride,
                      const void* weight, int w_dtype, void* out,
                      int64_t rows, int64_t D, float eps, void* stream);

/* ---------------------------------------------------------------------
 * Full-attention layers: the hybrid trunk's attention layers and the MTP
 * draft head (mtp.py:160-194 stacks the trunk's own full-attention
 * DecoderLayer after `fc`).  Those layers run mlx-lm's qwen3_5 Attention:
 * q_proj gives q and an output gate per head, q_norm / k_norm are RMSNorms
 * over the head dim, a rotary embedding covers the first
 * partial_rotary_factor * head_dim dims, scaled dot-product attention over a
 * KV cache ([B, Hkv, L, D], mlx-lm's KVCache layout), and the output is
 * multiplied by sigmoid(gate) before o_proj.  bf16 activations throughout.
 * --------------------------------------------------------------------- */

/*
 * q/k norm, rotary embedding and cache append for T new tokens per row:
 *   qg       [B,T,Hq,2D]   q_proj output, per head q then gate; qg_ld
 *            elements from one token to the next (0 = 2*Hq*D)
 *   k_new    [B,T,Hkv,D];  v_new [B,T,Hkv,D]; token stride kv_ld (0 = Hkv*D)
 *            (so q|gate, k and v may be column slices of one fused GEMM output)
 *   q_norm_w, k_norm_w [D] (w_dtype); y = x / sqrt(mean(x^2) + eps) * w,
 *            rounded to bf16 before the rotation
 *   pos0     [B] int32 device: each row's cache length before this call
 *            (= position of its first new token); clamped to [0, cap - T]
 *   q_out    [B,T,Hq,D];  k_cache, v_cache [B,Hkv,cap,D]
 *   rot      rotated dims (rotate-half pairs d, d + rot/2), angle
 *            pos * rope_base^(-2i/rot) for i = d mod rot/2
 * Requires D in {128, 256}.
 */
int gdn_attn_qk(const void* qg, int64_t qg_ld, const void* k_new, const void* v_new, int64_t kv_ld,
                const void* q_norm_w, const void* k_norm_w, int w_dtype, float eps,
                const int32_t* pos0, void* q_out, void* k_cache, void* v_cache, int64_t B,
                int64_t T, int64_t Hq, int64_t Hkv, int64_t D, int64_t cap, int64_t rot,
                float rope_base, void* stream);

/* Workspace bytes gdn_attn_fwd needs for n_split > 1 (0 for n_split == 1). */
size_t gdn_attn_workspace_bytes(int64_t B, int64_t T, int64_t Hq, int64_t Hkv, int64_t D,
                                int64_t n_split);

/*
 * Causal GQA attention of the T new tokens of each row over its cache
 * (keys 0 .. pos0[b] + t for token t; q-head h reads kv-head h / (Hq/Hkv)):
 *   out[b,t,h] = softmax(scale * q . K^T) V, times sigmoid(gate) when qg is
 *   not NULL (gate = second half of head h in qg [B,T,Hq,2D], token stride
 *   qg_ld as in gdn_attn_qk).
 *   kv_len_max  host bound of pos0[b] + T over the rows, in [T, cap]
 *   n_split     key ranges per row processed by separate workgroups (decode
 *               with long caches); > 1 needs gdn_attn_workspace_bytes.
 * q, caches 16-byte aligned; out and qg 8-byte aligned.  D in {128, 256}.
 */
int gdn_attn_fwd(const void* q, const void* qg, int64_t qg_ld, const void* k_cache, const void* v_cache,
                 const int32_t* pos0, void* out, float scale, int64_t B, int64_t T, int64_t Hq,
                 int64_t Hkv, int64_t D, int64_t cap, int64_t kv_len_max, int64_t n_split,
                 void* workspace, size_t workspace_bytes, void* stream);

/* RMSNorm of bf16 rows (mlx nn.RMSNorm): y = h / sqrt(mean(h^2) + eps) * w
 * with h = x, or h = bf16(x + res) when res is not NULL (a residual add
 * fused in front; h is written to h_out when not NULL, which may alias x).
 * y's rows are y_ld elements apart (0 = D), e.g. one half of a
 * concatenation.  D a multiple of 8; pointers 16-byte aligned; y may alias x
 * when y_ld == D and h_out is NULL. */
int gdn_rms_norm(const void* x, const void* res, void* h_out, const void* w, int w_dtype, void* y,
                 int64_t y_ld, int64_t rows, int64_t D, float eps, void* stream);

/* The MLP activation: out[r, i] = silu(gate_up[r, i]) * gate_up[r, I + i]
 * (bf16; gate_up is one [rows, 2I] product of the gate and up projections). */
int gdn_silu_mul(const void* gate_up, void* out, int64_t rows, int64_t I, void* stream);

/* ---------------------------------------------------------------------
 * Decode-shape projections of the GatedDeltaNet mixer (in_proj,
 * dflash.py:348-350; norm(out, z) then out_proj, dflash.py:377-378) for at
 * most 64 rows, where the weight read bounds the GEMM.
 * --------------------------------------------------------------------- */

/* Workspace bytes of gdn_linear_decode (0 for shapes it does not take): a
 * 16 KiB region of 32-bit tickets, one per 64-column output tile (N up to
 * 262144), then the fp32 partials of the K slices.  The ticket region must be
 * zero before the first call; every call leaves it zero, so one workspace,
 * sized for the largest shape, serves calls of any shape in turn.  Calls that
 * overlap (several streams) need one workspace each. */
size_t gdn_linear_decode_workspace_bytes(int64_t M, int64_t N, int64_t K);

/*
 * out[M, N] = A[M, K] W[N, K]^T in bf16 with fp32 accumulation, 1 <= M <= 64,
 * K a multiple of 512, N a multiple of 8:
 *   gate == NULL  A = x (rows ldx elements apart);
 *   gate != NULL  A = gated RMSNorm of x per head of head_dim (64 or 128)
 *                 columns, with gdn_gated_rmsnorm's arithmetic and rounding:
 *                 n = bf16(x / sqrt(mean(x^2) + eps)), m = bf16(w n) (w bf16)
 *                 or w n (w fp32; NULL = ones), A = bf16(m silu(gate)); gate
 *                 rows ldg elements apart, w [head_dim].
 *   W [N, K] row-major; out rows ldo elements apart.
 * Strides are multiples of 8 elements; pointers 16-byte aligned.  The K
 * slices of one output tile are summed in slice order, so results do not
 * depend on scheduling.  With the norm fused it is faster than the separate
 * norm plus a library GEMM up to 16 rows, and slower beyond (at hidden 2048,
 * graph-replayed); without the norm the library GEMM is faster.
 */
int gdn_linear_decode(const void* x, int64_t ldx, const void* gate, int64_t ldg, const void* norm_w,
                      int norm_w_dtype, float eps, int64_t head_dim, const void* W, void* out,
                      int64_t ldo, int64_t M, int64_t N, int64_t K, void* workspace,
                      size_t workspace_bytes, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* GDN_H */
