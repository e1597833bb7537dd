/*
 * mamba_mi355x.h -- C ABI of libmamba_mi355x.so, the MI355X (gfx950) kernels of
 * the Mamba selective-scan inference path.
 *
 * Replaces, for this path, the reference's kernel boundary:
 *   mamba_metal/_loader.py:29-42        load_kernel() -> mx.fast.metal_kernel
 *   mamba_metal/selective_scan.py:12-77 the selective_scan_chunked binding and dispatch
 * and the MLX ops the model runs around the scan:
 *   mamba_metal/mamba_block.py:45-52,77,129   nn.Conv1d (causal depthwise) + SiLU
 *   mamba_metal/mamba_block.py:170-177        decode conv-window step
 *   mamba_metal/mamba_block.py:183-195        decode SSM step
 *   mamba_metal/kernels/pair_scan.metal:1-76  block-level (a, b) pair scan primitive
 *
 * Conventions (all entry points):
 *   - Plain device pointers, int64 sizes and int64 ELEMENT strides; no framework types.
 *   - The caller allocates every buffer (inputs, outputs, workspace) on the current
 *     HIP device; the library never allocates or frees device memory.
 *   - Work is enqueued on `stream` (a hipStream_t passed as void*; NULL = default
 *     stream); no entry point synchronizes the device or the stream.
 *   - Return MM_OK (0) on success.  Invalid arguments are rejected by host-only
 *     validation BEFORE any HIP call, with a negative mm_status; the message is in
 *     mm_last_error() (thread-local).  A failed launch returns MM_ERR_HIP.
 *   - Host state: the thread-local error string, and per-device caches of launch
 *     constants (CU count, resident workgroups per CU) that are computed once and
 *     published with atomic stores.  Thread-safe.  Calls on one stream are ordered;
 *     calls on different streams that share output buffers race, as any two kernels
 *     would.
 */
#ifndef MAMBA_MI355X_H
#define MAMBA_MI355X_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MM_ABI_VERSION 6
/* Largest d_state accepted: mamba_metal/selective_scan.py:9 (MAX_DSTATE = 64). */
#define MM_MAX_DSTATE 64

/* Element types.  fp32 and fp16 are the reference's (experiments/10-fp16/test_fp16.py:1-12);
 * bf16 is accepted as well. */
typedef enum mm_dtype { MM_F32 = 0, MM_F16 = 1, MM_BF16 = 2 } mm_dtype;

typedef enum mm_status {
  MM_OK = 0,
  MM_ERR_NULL_POINTER = -1, /* a required pointer is NULL                          */
  MM_ERR_SHAPE = -2,        /* a size is negative / inconsistent                   */
  MM_ERR_DSTATE = -3,       /* dstate < 1 or > MM_MAX_DSTATE (selective_scan.py:50) */
  MM_ERR_DTYPE = -4,        /* unknown dtype enum                                  */
  MM_ERR_LAYOUT = -5,       /* a stride pattern the kernels do not accept          */
  MM_ERR_WORKSPACE = -6,    /* workspace missing or smaller than required          */
  MM_ERR_HIP = -7           /* a HIP launch failed (message has hipGetErrorString) */
} mm_status;

/* Version of this ABI (MM_ABI_VERSION). */
int mm_abi_version(void);
/* Last error message of the calling thread ("" if none). */
const char* mm_last_error(void);
/* Name of an mm_status value. */
const char* mm_status_name(int status);

/* ------------------------------------------------------------------------- */
/* (a) Selective scan -- replaces the selective_scan_chunked dispatch of
 *     mamba_metal/selective_scan.py:62-77 (kernel selective_scan_chunked.metal:28-155).
 *
 *   delta' = delta_softplus ? (delta <= 20 ? log(1+exp(delta)) : delta) : delta
 *   h[n]   = exp(delta'*A[d,n]) * h[n] + delta'*u*B[b,n,t]      (h = 0 at t = 0)
 *   y      = (sum_n C[b,n,t]*h[n] + D[d]*u) * (z ? silu(z) : 1)
 *   state_out[b,d,n] = h[n] after t = seqlen-1
 * Arithmetic is fp32 for every dtype; y is stored in x_dtype, state_out in fp32
 * (selective_scan.py:73-74).  D and z are optional (NULL = feature off,
 * selective_scan.py:52-60).
 */

/* Device workspace (bytes) the scan needs: B/C repacked as fp32 for the kernel,
 * the per-(channel block) state carried between time segments, and the work-queue
 * counter and flags.  Depends on dim through the number of 32- and 64-channel blocks,
 * and for few blocks (dstate <= 16) includes the split scan's segment summaries.
 * The int32 at byte offset 4 of the workspace is a status word, cleared by every call:
 * nonzero afterwards means a segment gave up waiting for its predecessor's carried
 * state (a bounded wait that is not expected to expire) and y is not valid.  Read it
 * once the stream has finished the call. */
size_t mm_selective_scan_workspace_size(int64_t batch, int64_t dim, int64_t dstate,
                                        int64_t seqlen);

/* Reference-shaped entry point: every tensor row-major contiguous exactly as
 * selective_scan.py:36-44 lays them out -- u, delta, z, y (batch, dim, seqlen);
 * A (dim, dstate) fp32; B, C (batch, dstate, seqlen); D (dim,) fp32;
 * ssm_state_out (batch, dim, dstate) fp32.  D, z, ssm_state_out may be NULL. */
int mm_selective_scan_fwd(const void* u, const void* delta, const float* A, const void* B,
                          const void* C, const float* D, const void* z, void* y,
                          float* ssm_state_out, int64_t batch, int64_t dim, int64_t dstate,
                          int64_t seqlen, int32_t x_dtype, int32_t bc_dtype,
                          int32_t delta_softplus, void* workspace, size_t workspace_bytes,
                          void* stream);

/* Strided form: same computation on arbitrary element strides, so the model can
 * pass its (batch, seqlen, dim) activations without the transposed copies of
 * mamba_block.py:90-100.  Fast paths: time-contiguous (stride[2] == 1) or
 * channel-contiguous (stride[1] == 1) u/delta/z/y; any other pattern runs a
 * slower gather path.  state_out is always contiguous (batch, dim, dstate). */
typedef struct mm_scan_params {
  const void* u;            /* (batch, dim, seqlen), x_dtype                     */
  const void* delta;        /* (batch, dim, seqlen), x_dtype                     */
  const float* A;           /* (dim, dstate), fp32                               */
  const void* B;            /* (batch, dstate, seqlen), bc_dtype                 */
  const void* C;            /* (batch, dstate, seqlen), bc_dtype                 */
  const float* D;           /* (dim,), fp32; NULL = no skip term                 */
  const void* z;            /* (batch, dim, seqlen), x_dtype; NULL = no gate      */
  void* y;                  /* (batch, dim, seqlen), x_dtype, output              */
  float* state_out;         /* (batch, dim, dstate) contiguous fp32; NULL = skip */
  void* workspace;          /* >= mm_selective_scan_workspace_size() bytes, 256-byte aligned */
  size_t workspace_bytes;
  int64_t batch, dim, dstate, seqlen;
  int64_t u_stride[3];      /* element strides in (batch, dim, time) order       */
  int64_t delta_stride[3];
  int64_t z_stride[3];
  int64_t y_stride[3];
  int64_t B_stride[3];      /* (batch, dstate, time)                             */
  int64_t C_stride[3];
  int64_t A_stride[2];      /* (dim, dstate)                                     */
  int64_t D_stride;
  int32_t x_dtype;          /* mm_dtype of u, delta, z, y                        */
  int32_t bc_dtype;         /* mm_dtype of B, C                                  */
  int32_t delta_softplus;   /* nonzero: apply softplus to delta                  */
  int32_t handoff_timeout_us; /* bound (microseconds) of a time segment's wait for its
                               predecessor's carried state; 0 = the default, 2 s.  The
                               wait always ends well before (a segment is claimed only
                               after its predecessor); the bound keeps every wave's exit
                               finite.  A wait that expires sets the status bits below
                               and the call's y is not valid.                      */
  int32_t* status;          /* optional device int32 (NULL = none): the kernel ORs
                               MM_SCAN_STATUS_* bits into it when y is not valid.
                               The library never clears it, so one word can collect
                               the outcome of many calls (e.g. every layer of a
                               prefill); the caller zeroes it and reads it after
                               the stream has finished. */
} mm_scan_params;

/* Bits of mm_scan_params.status (and of the workspace status word). */
#define MM_SCAN_STATUS_HANDOFF_TIMEOUT 1 /* a segment gave up waiting for the carried state */

int mm_selective_scan_fwd_strided(const mm_scan_params* p, void* stream);

/* Allocation-free form of mm_selective_scan_fwd.  No counterpart in the reference: it is
 * for callers that cannot allocate device memory (code under HIP graph capture, tight
 * serving loops, harnesses that forbid hipMalloc).  Same arguments, semantics and
 * results as mm_selective_scan_fwd, without the workspace: the library keeps one scan
 * workspace of MM_SCAN_SCRATCH_BYTES per device in a static device array, held until
 * the process ends.  When mm_selective_scan_workspace_size exceeds
 * MM_SCAN_SCRATCH_BYTES only because of the split scan's segment summaries, the call runs
 * the chained scan (the same result up to fp32 rounding); shapes whose chained share
 * exceeds it too are rejected with MM_ERR_WORKSPACE (host-side, before any HIP call).
 * It calls no allocating routine.  Every call on a device uses that device's
 * array, so calls that overlap in time on one device race (order them on one stream).
 * `status` is optional (NULL = none), a device int32 as mm_scan_params.status: the call
 * ORs MM_SCAN_STATUS_* bits into it when its y is not valid; never cleared by the
 * library.  The array's device address is looked up on the first call on each device
 * (hipGetSymbolAddress, which does not allocate). */
#define MM_SCAN_SCRATCH_BYTES (32u << 20)
int mm_selective_scan_fwd_noalloc(const void* u, const void* delta, const float* A,
                                  const void* B, const void* C, const float* D, const void* z,
                                  void* y, float* ssm_state_out, int64_t batch, int64_t dim,
                                  int64_t dstate, int64_t seqlen, int32_t x_dtype,
                                  int32_t bc_dtype, int32_t delta_softplus, int32_t* status,
                                  void* stream);

/* ------------------------------------------------------------------------- */
/* (b) Causal depthwise conv1d over time, channels-last -- replaces
 *     nn.Conv1d(groups=d_inner, padding=d_conv-1)[:, :L] + nn.silu of
 *     mamba_block.py:45-52,77-78,129-130, and the conv-state slice of
 *     mamba_block.py:118-127.
 *
 *   out[b,t,c] = act(bias[c] + sum_{k<width} w[c,k] * x[b, t-(width-1)+k, c]),  x[<0] = 0
 *   conv_state_out[b,c,k] = x[b, seqlen-width+k, c]  (0 where the index is < 0)
 * x/out strides are (batch, time, channel) in elements; weight is (dim, width)
 * with strides w_stride (the HF/torch (dim, 1, width) tensor viewed 2-D).
 * bias and conv_state_out ((batch, dim, width) contiguous, x_dtype) may be NULL.
 * width <= 8. */
int mm_causal_conv1d_fwd(const void* x, const void* weight, const void* bias, void* out,
                         void* conv_state_out, int64_t batch, int64_t seqlen, int64_t dim,
                         int64_t width, const int64_t x_stride[3], const int64_t out_stride[3],
                         const int64_t w_stride[2], int32_t x_dtype, int32_t w_dtype,
                         int32_t apply_silu, void* stream);

/* ------------------------------------------------------------------------- */
/* (c) O(1) decode step, in two kernels around the x_proj GEMM.
 *
 * Conv window step -- replaces mamba_block.py:170-177:
 *   conv_state[b,c,:] <- (conv_state[b,c,1:], x[b,c])          (in place)
 *   out[b,c] = act(bias[c] + sum_k w[c,k] * conv_state[b,c,k])
 * conv_state is (batch, dim, width) contiguous in state_dtype; x/out are
 * (batch, dim) with batch strides x_stride_b/out_stride_b and unit channel
 * stride, x_dtype.  bias may be NULL. */
int mm_decode_conv_step(void* conv_state, const void* x, const void* weight, const void* bias,
                        void* out, int64_t batch, int64_t dim, int64_t width,
                        int64_t x_stride_b, int64_t out_stride_b, const int64_t w_stride[2],
                        int32_t state_dtype, int32_t x_dtype, int32_t w_dtype,
                        int32_t apply_silu, void* stream);

/* SSM step -- replaces mamba_block.py:183-195 (fused: softplus, discretise,
 * state update, C contraction, D skip, SiLU(z) gate):
 *   dt' = softplus(dt + dt_bias)          (logaddexp form, mamba_block.py:184)
 *   h[b,c,n] <- exp(dt'*A[c,n]) * h[b,c,n] + dt'*x[b,c]*B[b,n]   (in place, fp32)
 *   y[b,c] = (sum_n h[b,c,n]*C[b,n] + D[c]*x[b,c]) * silu(z[b,c])
 * ssm_state (batch, dim, dstate) contiguous fp32.  x, dt, z, y: (batch, dim),
 * x_dtype, batch strides given, unit channel stride.  B, C: (batch, dstate),
 * x_dtype, batch strides given, unit state stride.  A (dim, dstate) contiguous
 * fp32; dt_bias (dim,), D (dim,) fp32 and z may be NULL. */
int mm_decode_ssm_step(float* ssm_state, const void* x, const void* dt, const float* dt_bias,
                       const float* A, const void* B, const void* C, const float* D,
                       const void* z, void* y, int64_t batch, int64_t dim, int64_t dstate,
                       int64_t x_stride_b, int64_t dt_stride_b, int64_t B_stride_b,
                       int64_t C_stride_b, int64_t z_stride_b, int64_t y_stride_b,
                       int32_t x_dtype, int32_t dt_softplus, void* stream);

/* Fused SSM step with the dt projection folded in -- replaces mamba_block.py:183-195
 * together with the dt_proj Linear of :183:
 *   dt[b,c] = softplus(dt_bias[c] + sum_r dt_in[b,r] * dt_weight[c,r])
 * then the update of mm_decode_ssm_step.  dt_in (batch, rank) with batch stride
 * dt_stride_b and unit stride (the dt slice of x_proj's output); dt_weight (dim, rank)
 * with row stride w_stride_c, dt_bias (dim,) in w_dtype (may be NULL); rank <= 256.
 * Other arguments as mm_decode_ssm_step. */
int mm_decode_ssm_step_dtproj(float* ssm_state, const void* x, const void* dt_in,
                              const void* dt_weight, const void* dt_bias, const float* A,
                              const void* B, const void* C, const float* D, const void* z,
                              void* y, int64_t batch, int64_t dim, int64_t dstate, int64_t rank,
                              int64_t x_stride_b, int64_t dt_stride_b, int64_t w_stride_c,
                              int64_t B_stride_b, int64_t C_stride_b, int64_t z_stride_b,
                              int64_t y_stride_b, int32_t x_dtype, int32_t w_dtype, void* stream);

/* ------------------------------------------------------------------------- */
/* Fused residual add + RMSNorm -- replaces `x + mixer(...)` followed by the next
 * layer's nn.RMSNorm (mamba_model.py:40,48,53,57,69):
 *   resid[r,:] += add[r,:]           (skipped when add is NULL; kept in x_dtype)
 *   out[r,:]    = resid[r,:] * rsqrt(mean(resid[r,:]^2) + eps) * weight
 * rows x dim, row strides given, unit column stride; weight (dim,) in w_dtype;
 * dim <= 8192. */
int mm_add_rmsnorm(void* resid, const void* add, const void* weight, void* out, int64_t rows,
                   int64_t dim, int64_t resid_stride, int64_t add_stride, int64_t out_stride,
                   float eps, int32_t x_dtype, int32_t w_dtype, void* stream);

/* ------------------------------------------------------------------------- */
/* Decode-step GEMM with fused epilogues -- replaces the nn.Linear projections of
 * MambaBlock.step (in_proj mamba_block.py:166, x_proj :180, out_proj :196) and the
 * tied LM head (mamba_model.py:78) at decode batch M <= 64:
 *   acc[m, n] = sum_k x[m, k] * w[n, k]          (w is nn.Linear's (N, K) weight)
 * epilogue MM_LIN_STORE: y[m, n] = acc.
 * epilogue MM_LIN_RESID: resid[m, n] = resid[m, n] + round(acc)  (out_proj followed
 *   by the residual add of mamba_model.py:48; y unused).
 * epilogue MM_LIN_RESID_NORM: as MM_LIN_RESID, then the next RMSNorm of the updated
 *   rows (mamba_model.py:40,48,69): norm_out[m, :] = resid[m, :] *
 *   rsqrt(mean(resid[m, :]^2) + eps) * norm_w (norm_w in dtype; one launch fewer
 *   than RESID + mm_add_rmsnorm).
 * epilogue MM_LIN_CONV:  in_proj followed by the conv-window step of
 *   mamba_block.py:172-179 on columns [0, n_conv): x = round(acc); conv_state
 *   (M, n_conv, 4) contiguous shifts in place; conv_out[m, n] = silu(conv_b[n] +
 *   sum_j conv_w[n, j] * window_j); columns >= n_conv store y[m, n - n_conv] = acc.
 * w is passed PACKED (mm_pack_linear_weight, once per weight).  f16 / bf16 only
 * (one dtype for every tensor); K a multiple of 64; ldx >= K a multiple of 8; x
 * and w_packed 16-byte aligned.  Narrow N splits K across workgroups: fp32
 * partials go to the workspace (mm_decode_linear_workspace_size bytes, 16-byte
 * aligned, no initial contents needed) and a second kernel sums them; calls that
 * overlap in time must not share a workspace. */
typedef enum mm_linear_epilogue {
  MM_LIN_STORE = 0,
  MM_LIN_RESID = 1,
  MM_LIN_CONV = 2,
  MM_LIN_RESID_NORM = 3
} mm_linear_epilogue;

typedef struct mm_linear_params {
  const void* x;          /* (M, K), row stride ldx */
  const void* w_packed;   /* mm_pack_linear_weight output for the (N, K) weight */
  void* y;                /* (M, N) row stride ldy (CONV: (M, N - n_conv)) */
  void* resid;            /* RESID: (M, N) row stride ldr */
  void* conv_state;       /* CONV: (M, n_conv, 4) contiguous */
  const void* conv_w;     /* CONV: (n_conv, 4) contiguous */
  const void* conv_b;     /* CONV: (n_conv,) or NULL */
  void* conv_out;         /* CONV: (M, n_conv) row stride ldc */
  const void* norm_w;     /* RESID_NORM: (N,) */
  void* norm_out;         /* RESID_NORM: (M, N) row stride ldn */
  void* workspace;        /* split-K counters + partial tiles (may be NULL if size 0) */
  size_t workspace_bytes;
  int64_t M, N, K;
  int64_t ldx, ldy, ldr, ldc, ldn;
  int64_t n_conv;
  float eps;              /* RESID_NORM */
  int32_t dtype;          /* MM_F16 or MM_BF16 */
  int32_t epilogue;       /* mm_linear_epilogue */
  /* Optional input RMSNorm (NULL: off).  When set, x holds the raw residual rows
   * and the product uses round(x * rsqrt(mean(x^2) + x_eps) * x_norm_w) -- the
   * MambaResidualBlock.step norm of mamba_model.py:57 evaluated in the operand load,
   * bit-identical to mm_add_rmsnorm's output.  (K,) in dtype, 16-byte aligned;
   * M <= 8, K <= 4096 and N <= 16384. */
  const void* x_norm_w;
  float x_eps;
  int32_t reserved;       /* must be 0 */
} mm_linear_params;

/* Bytes of the packed copy of an (N, K) weight: ceil(N/32)*32 * K elements. */
size_t mm_packed_linear_weight_bytes(int64_t N, int64_t K, int32_t dtype);
/* Repack w (N, K), row stride ldw, into the decode GEMM's operand order. */
int mm_pack_linear_weight(const void* w, void* packed, int64_t N, int64_t K, int64_t ldw,
                          int32_t dtype, void* stream);
/* Workspace bytes mm_decode_linear needs for (M, N, K); 0 when it needs none. */
size_t mm_decode_linear_workspace_size(int64_t M, int64_t N, int64_t K);
int mm_decode_linear(const mm_linear_params* params, void* stream);

/* in_proj + conv-window step + x_proj of one decode step -- replaces the
 * in_proj -> conv window -> x_proj chain of MambaBlock.step (mamba_block.py:166-182):
 * runs mm_decode_linear(params) (epilogue MM_LIN_CONV), then
 * xp_y[m, n] = round(sum_k conv_out[m, k] * W_x[n, k]) for n < xp_n, k < n_conv, with
 * xp_w_packed the mm_pack_linear_weight copy of the (xp_n, n_conv) x_proj weight and
 * xp_y rows of stride ld_xp in params->dtype.  Where the in_proj shape allows (4-wave
 * K-resident workgroups, no input RMSNorm, workgroup columns on one side of n_conv,
 * xp_n <= 256 and a multiple of 4) the x_proj products are taken in in_proj's conv
 * epilogue from the conv outputs still on chip, as fp32 partials per workgroup,
 * summed in a fixed order by one small kernel; otherwise the two GEMMs run one after
 * the other.  The workspace (params->workspace) must hold
 * mm_decode_in_proj_xproj_workspace_size bytes, 16-byte aligned. */
size_t mm_decode_in_proj_xproj_workspace_size(int64_t M, int64_t N, int64_t K, int64_t n_conv,
                                              int64_t xp_n);
int mm_decode_in_proj_xproj(const mm_linear_params* params, const void* xp_w_packed,
                            int64_t xp_n, void* xp_y, int64_t ld_xp, void* stream);

/* LM head + greedy choice of one decode step -- replaces the tied head
 * (mamba_model.py:78, logits = h @ E^T) followed by generate_fast's greedy
 * `mx.argmax(logits[:, -1, :])` (generate.py:91-93): runs mm_decode_linear(params)
 * (epilogue MM_LIN_STORE: the logits y are stored as there) and writes ids[m] = the
 * column of the largest stored y[m, :] (lowest column on ties, a NaN beats every
 * number: mm_argmax_rows's result on the stored logits).  For the wide N of a head the
 * per-workgroup maxima are taken in the GEMM's epilogue and one small kernel picks
 * among them; otherwise mm_argmax_rows runs on y.  ids int64 (M,), 8-byte aligned;
 * params->workspace must hold mm_decode_head_argmax_workspace_size bytes. */
size_t mm_decode_head_argmax_workspace_size(int64_t M, int64_t N, int64_t K);
int mm_decode_head_argmax(const mm_linear_params* params, int64_t* ids, void* stream);

/* mm_decode_head_argmax, then the next step's embedding lookup -- replaces generate.py's
 * feeding of the chosen ids back through the embedding (mamba_model.py:75,
 * self.embedding(input_ids)): rows[m, k] = table[ids[m], k] for k < params->K.  table is
 * the (N, K) embedding matrix the head is tied to, row-major with row stride ld_table;
 * rows has row stride ld_rows; both 2-byte elements, strides multiples of 8 (>= K),
 * 16-byte aligned, rows not overlapping x or y.  On the fused head path the copy runs
 * in the kernel that picks the ids. */
int mm_decode_head_argmax_embed(const mm_linear_params* params, int64_t* ids, const void* table,
                                int64_t ld_table, void* rows, int64_t ld_rows, void* stream);

/* ------------------------------------------------------------------------- */
/* Prefill projection GEMM for short K -- replaces the dt projection of the parallel
 * prefill (MambaBlock.prefill, mamba_block.py:136: dt_proj with its bias, K = dt_rank):
 *   y[m, n] = round(sum_k x[m, k] * w[n, k] + bias[n])     (fp32 accumulation)
 * x (M, K) row stride ldx; w nn.Linear's (N, K) weight, row stride ldw (not packed);
 * bias (N,) or NULL; y (M, N) row stride ldy.  f16 / bf16, one dtype for every tensor;
 * K a multiple of 16; ldx and ldw multiples of 8; x and w 16-byte aligned.  Operands go
 * straight from memory to the matrix cores: any K is computed correctly, but only short
 * K (up to a few hundred) is faster than a library GEMM.  No workspace. */
int mm_prefill_linear(const void* x, const void* w, const void* bias, void* y, int64_t M,
                      int64_t N, int64_t K, int64_t ldx, int64_t ldw, int64_t ldy, int32_t dtype,
                      void* stream);

/* ------------------------------------------------------------------------- */
/* Greedy token choice -- replaces `mx.argmax(logits[:, -1, :], axis=-1)` of
 * generate_fast (generate.py:91-93): out[r] = index of the largest x[r, 0:n]
 * (lowest index on ties, a NaN beats every number).  x rows of stride >= n in
 * dtype; out int64 (rows,). */
int mm_argmax_rows(const void* x, int64_t rows, int64_t n, int64_t stride, int32_t dtype,
                   int64_t* out, void* stream);

/* ------------------------------------------------------------------------- */
/* Pair-scan primitive -- replaces mamba_metal/kernels/pair_scan.metal:1-76
 * (dispatched by experiments/05-pair-scan/pair_scan.py:23-33), without its
 * n <= 1024 limit: inclusive scan of (a, b) under (a2,b2)o(a1,b1) =
 * (a2*a1, a2*b1 + b2).  a_out[i] = prod_{k<=i} a[k]; h_out[i] = h_i with
 * h_i = a_i*h_{i-1} + b_i, h_{-1} = 0.  fp32, contiguous, a_out may be NULL. */
int mm_pair_scan(const float* a, const float* b, float* a_out, float* h_out, int64_t n,
                 void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MAMBA_MI355X_H */
