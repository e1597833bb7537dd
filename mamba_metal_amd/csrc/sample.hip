// Greedy token selection: mm_argmax_rows.
//
// Replaces the argmax of generate_fast's greedy step (mamba_metal/generate.py:91-93,
// mx.argmax over the vocabulary of the last logits row).  One workgroup per row
// streams the row once (16-byte loads when the row allows it); ties go to the lowest
// index and a NaN counts as larger than any number -- torch.argmax's conventions, so
// the chosen ids match the framework the caller would otherwise use.
#include "mm_common.h"

namespace mm {
namespace sample {

constexpr int kThreads = 1024;
constexpr int kUnroll = 4;  // independent loads in flight per thread

// a better than b: NaN first, then larger value, then lower index.
__device__ __forceinline__ bool better(float av, int64_t ai, float bv, int64_t bi) {
  const bool an = av != av, bn = bv != bv;
  if (an != bn) return an;
  if (!an && av != bv) return av > bv;
  return ai < bi;
}

// Running best of one thread, whose elements arrive in increasing index order: a
// later element replaces the best only when strictly larger, or when it is the first
// NaN, or when the thread has none yet (bi < 0).
__device__ __forceinline__ void take(float f, int32_t i, bool valid, float& bv, int32_t& bi) {
  const bool t = valid && (bi < 0 || f > bv || (f != f && bv == bv));
  bv = t ? f : bv;
  bi = t ? i : bi;
}

// One workgroup per row.  VEC: 16-byte chunks of 8 elements, chunk c = tid + 1024 j;
// each iteration issues kUnroll chunk loads (clamped to the row: a chunk past the end
// re-reads chunk 0 and is masked) before comparing any of them.
template <int DT, bool VEC>
__global__ __launch_bounds__(kThreads) void argmax_kernel(const void* __restrict__ x, int64_t n,
                                                          int64_t stride, int64_t* __restrict__ out) {
  using T = typename Ty<DT>::T;
  using V8 = typename Ty<DT>::V8;
  __shared__ float s_v[kThreads / 64];
  __shared__ int32_t s_i[kThreads / 64];
  const int tid = threadIdx.x;
  const T* row = static_cast<const T*>(x) + static_cast<int64_t>(blockIdx.x) * stride;
  float bv = -__builtin_inff();
  int32_t bi = -1;
  const int32_t n32 = static_cast<int32_t>(n);
  if constexpr (VEC) {
    const int32_t nch = n32 / 8;
    for (int32_t c0 = tid; c0 < nch; c0 += kThreads * kUnroll) {
      V8 v[kUnroll];
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) {
        const int32_t c = c0 + u * kThreads;
        v[u] = *reinterpret_cast<const V8*>(row + 8 * static_cast<int64_t>(c < nch ? c : 0));
      }
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) {
        const int32_t c = c0 + u * kThreads;
#pragma unroll
        for (int k = 0; k < 8; ++k) take(Ty<DT>::f(v[u][k]), 8 * c + k, c < nch, bv, bi);
      }
    }
  } else {
    constexpr int U = 2 * kUnroll;
    for (int32_t i0 = tid; i0 < n32; i0 += kThreads * U) {
      T v[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int32_t i = i0 + u * kThreads;
        v[u] = row[i < n32 ? i : 0];
      }
#pragma unroll
      for (int u = 0; u < U; ++u) take(Ty<DT>::f(v[u]), i0 + u * kThreads, i0 + u * kThreads < n32, bv, bi);
    }
  }
  // Across threads: full comparison (value, then index); a thread with no element
  // carries index n, which loses to every real element.
  // Indices fit int32 (n <= 2^30, checked on the host) and move between lanes as raw bits.
  int32_t bl = bi < 0 ? n32 : bi;
  if (bi < 0) bv = -__builtin_inff();
  auto xchg = [](float& v, int32_t& i, int off) __attribute__((always_inline)) {
    const float ov = lane_xor(v, off);
    const int32_t oi = __float_as_int(lane_xor(__int_as_float(i), off));
    if (better(ov, oi, v, i)) {
      v = ov;
      i = oi;
    }
  };
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) xchg(bv, bl, off);
  if ((tid & 63) == 0) {
    s_v[tid >> 6] = bv;
    s_i[tid >> 6] = bl;
  }
  __syncthreads();
  if (tid < 64) {  // all of wave 0
    bv = tid < kThreads / 64 ? s_v[tid] : -__builtin_inff();
    bl = tid < kThreads / 64 ? s_i[tid] : n32;
#pragma unroll
    for (int off = 8; off > 0; off >>= 1) xchg(bv, bl, off);
    if (tid == 0) out[blockIdx.x] = bl;
  }
}

}  // namespace sample
}  // namespace mm

extern "C" {

int mm_argmax_rows(const void* x, int64_t rows, int64_t n, int64_t stride, int32_t dtype,
                   int64_t* out, void* stream) {
  using namespace mm;
  using namespace mm::sample;
  clear_error();
  if (!x || !out) return fail(MM_ERR_NULL_POINTER, "x and out are required");
  if (rows < 0 || n < 1) return fail(MM_ERR_SHAPE, "rows must be >= 0 and n >= 1");
  if (rows > 0x7fffffff || n > 0x3fffffff) return fail(MM_ERR_SHAPE, "too many rows or columns");
  if (stride < n) return fail(MM_ERR_LAYOUT, "row stride smaller than n");
  if (!valid_dtype(dtype)) return fail(MM_ERR_DTYPE, "bad dtype %d", dtype);
  if (rows == 0) return MM_OK;
  const int64_t es = dtype_size(dtype);
  const bool vec = n % 8 == 0 && (stride * es) % (8 * es) == 0 && aligned(x, 8 * es);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const dim3 grid(static_cast<unsigned>(rows));
#define MM_AM(D)                                                                          \
  if (vec)                                                                                \
    hipLaunchKernelGGL((argmax_kernel<D, true>), grid, dim3(kThreads), 0, s, x, n, stride, out); \
  else                                                                                    \
    hipLaunchKernelGGL((argmax_kernel<D, false>), grid, dim3(kThreads), 0, s, x, n, stride, out)
  switch (dtype) {
    case MM_F32: MM_AM(MM_F32); break;
    case MM_F16: MM_AM(MM_F16); break;
    default: MM_AM(MM_BF16); break;
  }
#undef MM_AM
  return check_launch("argmax_rows");
}

}  // extern "C"
