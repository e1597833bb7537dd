// (a, b) pair-scan primitive: mm_pair_scan.
//
// Replaces mamba_metal/kernels/pair_scan.metal:1-76 (Hillis-Steele over 32-lane
// simdgroups + a threadgroup bridge, n <= 1024).  Here a wave64 scan is built
// from DPP lane moves: row_shr:1/2/4/8 inside each 16-lane row, then
// row_bcast:15 / row_bcast:31 across rows (both GFX9-family DPP controls that
// gfx950 keeps); 16 waves bridge through LDS; a running carry extends the scan
// over arbitrary n, chunk by chunk.  The operator is
//   (a2, b2) o (a1, b1) = (a2*a1, a2*b1 + b2),  identity (1, 0)
// and lanes with no source get the identity through update_dpp's `old` value.
#include "mm_common.h"

namespace mm {
namespace pscan {

constexpr int kThreads = 1024;
constexpr int kWaves = kThreads / 64;

template <int CTRL, int ROW_MASK>
__device__ __forceinline__ void dpp_combine(float& a, float& b) {
  const float pa = __int_as_float(__builtin_amdgcn_update_dpp(
      __float_as_int(1.0f), __float_as_int(a), CTRL, ROW_MASK, 0xf, false));
  const float pb = __int_as_float(__builtin_amdgcn_update_dpp(
      __float_as_int(0.0f), __float_as_int(b), CTRL, ROW_MASK, 0xf, false));
  b = __builtin_fmaf(a, pb, b);
  a = a * pa;
}

// Inclusive pair scan across the 64 lanes of a wave.
__device__ __forceinline__ void wave_pair_scan(float& a, float& b) {
  dpp_combine<0x111, 0xf>(a, b);  // row_shr:1
  dpp_combine<0x112, 0xf>(a, b);  // row_shr:2
  dpp_combine<0x114, 0xf>(a, b);  // row_shr:4
  dpp_combine<0x118, 0xf>(a, b);  // row_shr:8
  dpp_combine<0x142, 0xa>(a, b);  // row_bcast:15 -> rows 1, 3
  dpp_combine<0x143, 0xc>(a, b);  // row_bcast:31 -> rows 2, 3
}

__global__ __launch_bounds__(kThreads) void pair_scan_kernel(const float* __restrict__ a_in,
                                                             const float* __restrict__ b_in,
                                                             float* __restrict__ a_out,
                                                             float* __restrict__ h_out,
                                                             int64_t n) {
  __shared__ float wa[kWaves], wb[kWaves];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  float ca = 1.0f, cb = 0.0f;  // composition of every element before this chunk
  for (int64_t base = 0; base < n; base += kThreads) {
    const int64_t i = base + tid;
    float a = i < n ? a_in[i] : 1.0f;
    float b = i < n ? b_in[i] : 0.0f;
    wave_pair_scan(a, b);
    if (lane == 63) {
      wa[wave] = a;
      wb[wave] = b;
    }
    __syncthreads();
    float pa = 1.0f, pb = 0.0f;  // composition of earlier waves of this chunk
    float ta = 1.0f, tb = 0.0f;  // composition of all waves of this chunk
    for (int w = 0; w < kWaves; ++w) {
      const float xa = wa[w], xb = wb[w];
      if (w < wave) {
        pb = __builtin_fmaf(xa, pb, xb);
        pa = xa * pa;
      }
      tb = __builtin_fmaf(xa, tb, xb);
      ta = xa * ta;
    }
    const float hb = __builtin_fmaf(pa, cb, pb);  // h just before this wave
    const float ha = pa * ca;
    if (i < n) {
      if (a_out) a_out[i] = a * ha;
      h_out[i] = __builtin_fmaf(a, hb, b);
    }
    cb = __builtin_fmaf(ta, cb, tb);
    ca = ta * ca;
    __syncthreads();
  }
}

}  // namespace pscan
}  // namespace mm

extern "C" {

int mm_pair_scan(const float* a, const float* b, float* a_out, float* h_out, int64_t n,
                 void* stream) {
  using namespace mm;
  clear_error();
  if (!a || !b || !h_out) return fail(MM_ERR_NULL_POINTER, "a, b and h_out are required");
  if (n < 0) return fail(MM_ERR_SHAPE, "negative n=%lld", (long long)n);
  if (n == 0) return MM_OK;
  hipLaunchKernelGGL(pscan::pair_scan_kernel, dim3(1), dim3(pscan::kThreads), 0,
                     static_cast<hipStream_t>(stream), a, b, a_out, h_out, n);
  return check_launch("pair_scan");
}

}  // extern "C"
