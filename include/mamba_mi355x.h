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
 *   - No global mutable state besides the thread-local error string: thread-safe.
 *     Calls on one stream are ordered; calls on different streams that share
 *     output buffers race, as any two kernels would.
 */
#ifndef MAMBA_MI355X_H
#define MAMBA_MI355X_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MM_ABI_VERSION 1
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
 * counter and flags.  Depends on dim through the number of 64-channel blocks. */
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
  int32_t reserved;         /* must be 0                                         */
} mm_scan_params;

int mm_selective_scan_fwd_strided(const mm_scan_params* p, void* stream);

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
