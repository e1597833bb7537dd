// O(1) decode SSM step: mm_decode_ssm_step.
//
// Replaces the elementwise tail of MambaBlock.step (mamba_metal/mamba_block.py:183-195):
// softplus(dt) (MLX logaddexp form, :184), a = exp(dt*A), b = (dt*x)*B, h = a*h + b,
// y = sum_n h*C + D*x, y *= silu(z) -- about twenty lazy MLX ops in the reference --
// as one kernel that reads and rewrites the resident fp32 state in place.
//
// One thread per (batch, channel); the workgroup covers 256 channels of ONE batch
// row so B[b, :] and C[b, :] are wave-uniform (scalar loads, SGPR operands).  The
// state row (dstate fp32, contiguous) is read and written with 16-byte accesses:
// the kernel is HBM-bound on 2 x 4 x dstate bytes of state per (b, c).
#include "mm_common.h"

namespace mm {
namespace dec {

constexpr int kBlock = 256;

struct Params {
  float* h;
  const void* x;
  const void* dt;
  const float* dt_bias;
  const float* A;
  const void* B;
  const void* C;
  const float* D;
  const void* z;
  void* y;
  int64_t dim, dstate, xsb, dtsb, Bsb, Csb, zsb, ysb;
  int32_t softplus;
};

template <int DT, int NS>
__global__ __launch_bounds__(kBlock) void ssm_step_kernel(const Params p) {
  const int64_t c = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x;
  const int64_t b = blockIdx.y;
  if (c >= p.dim) return;
  const int N = static_cast<int>(p.dstate);

  const float xv = ld<DT>(p.x, b * p.xsb + c);
  float dtv = ld<DT>(p.dt, b * p.dtsb + c);
  if (p.dt_bias) dtv += p.dt_bias[c];
  if (p.softplus) dtv = softplus_full(dtv);
  const float du = dtv * xv;
  const float dtl = dtv * kLog2e;

  float* hp = p.h + (b * p.dim + c) * p.dstate;
  const float* Ap = p.A + c * p.dstate;
  float acc = 0.0f;
  if (N == NS && (NS % 4) == 0) {
    // Full rows: 16-byte state / A accesses.
#pragma unroll
    for (int n4 = 0; n4 < NS; n4 += 4) {
      float4 hv = *reinterpret_cast<const float4*>(hp + n4);
      const float4 av = *reinterpret_cast<const float4*>(Ap + n4);
      float hs[4] = {hv.x, hv.y, hv.z, hv.w};
      const float as[4] = {av.x, av.y, av.z, av.w};
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const int n = n4 + k;
        const float a = exp2_hw(dtl * as[k]);
        hs[k] = __builtin_fmaf(a, hs[k], du * ld<DT>(p.B, b * p.Bsb + n));
        acc = __builtin_fmaf(hs[k], ld<DT>(p.C, b * p.Csb + n), acc);
      }
      *reinterpret_cast<float4*>(hp + n4) = make_float4(hs[0], hs[1], hs[2], hs[3]);
    }
  } else {
#pragma unroll
    for (int n = 0; n < NS; ++n) {
      if (n < N) {
        const float a = exp2_hw(dtl * Ap[n]);
        const float hn = __builtin_fmaf(a, hp[n], du * ld<DT>(p.B, b * p.Bsb + n));
        hp[n] = hn;
        acc = __builtin_fmaf(hn, ld<DT>(p.C, b * p.Csb + n), acc);
      }
    }
  }
  if (p.D) acc = __builtin_fmaf(p.D[c], xv, acc);
  if (p.z) acc *= silu_f(ld<DT>(p.z, b * p.zsb + c));
  st<DT>(p.y, b * p.ysb + c, acc);
}

template <int DT>
void launch(const Params& p, int64_t batch, hipStream_t s) {
  const dim3 grid(static_cast<unsigned>(ceil_div(p.dim, kBlock)), static_cast<unsigned>(batch));
  const int64_t N = p.dstate;
  if (N <= 4)
    hipLaunchKernelGGL((ssm_step_kernel<DT, 4>), grid, dim3(kBlock), 0, s, p);
  else if (N <= 8)
    hipLaunchKernelGGL((ssm_step_kernel<DT, 8>), grid, dim3(kBlock), 0, s, p);
  else if (N <= 16)
    hipLaunchKernelGGL((ssm_step_kernel<DT, 16>), grid, dim3(kBlock), 0, s, p);
  else if (N <= 32)
    hipLaunchKernelGGL((ssm_step_kernel<DT, 32>), grid, dim3(kBlock), 0, s, p);
  else
    hipLaunchKernelGGL((ssm_step_kernel<DT, 64>), grid, dim3(kBlock), 0, s, p);
}

}  // namespace dec
}  // namespace mm

extern "C" {

int mm_decode_ssm_step(float* ssm_state, const void* x, const void* dt, const float* dt_bias,
                       const float* A, const void* B, const void* C, const float* D,
                       const void* z, void* y, int64_t batch, int64_t dim, int64_t dstate,
                       int64_t x_stride_b, int64_t dt_stride_b, int64_t B_stride_b,
                       int64_t C_stride_b, int64_t z_stride_b, int64_t y_stride_b,
                       int32_t x_dtype, int32_t dt_softplus, void* stream) {
  using namespace mm;
  using namespace mm::dec;
  clear_error();
  if (!ssm_state || !x || !dt || !A || !B || !C || !y)
    return fail(MM_ERR_NULL_POINTER, "ssm_state, x, dt, A, B, C and y are required");
  if (batch < 0 || dim < 0) return fail(MM_ERR_SHAPE, "negative size");
  if (batch > 65535) return fail(MM_ERR_SHAPE, "batch=%lld exceeds 65535", (long long)batch);
  if (dstate < 1 || dstate > MM_MAX_DSTATE)
    return fail(MM_ERR_DSTATE, "dstate=%lld outside [1, %d]", (long long)dstate, MM_MAX_DSTATE);
  if (!valid_dtype(x_dtype)) return fail(MM_ERR_DTYPE, "bad dtype %d", x_dtype);
  if (!aligned(ssm_state, 16) || !aligned(A, 16))
    return fail(MM_ERR_LAYOUT, "ssm_state and A must be 16-byte aligned");
  if (batch == 0 || dim == 0) return MM_OK;
  Params p;
  p.h = ssm_state;
  p.x = x;
  p.dt = dt;
  p.dt_bias = dt_bias;
  p.A = A;
  p.B = B;
  p.C = C;
  p.D = D;
  p.z = z;
  p.y = y;
  p.dim = dim;
  p.dstate = dstate;
  p.xsb = x_stride_b;
  p.dtsb = dt_stride_b;
  p.Bsb = B_stride_b;
  p.Csb = C_stride_b;
  p.zsb = z_stride_b;
  p.ysb = y_stride_b;
  p.softplus = dt_softplus ? 1 : 0;
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (x_dtype) {
    case MM_F32: launch<MM_F32>(p, batch, s); break;
    case MM_F16: launch<MM_F16>(p, batch, s); break;
    default: launch<MM_BF16>(p, batch, s); break;
  }
  return check_launch("decode_ssm_step");
}

}  // extern "C"
