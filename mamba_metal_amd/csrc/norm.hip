// Fused residual add + RMSNorm: mm_add_rmsnorm.
//
// Replaces, on the decode and prefill paths, the pair
//   x = x + mixer(...)                      (mamba_model.py:48, :53, :57)
//   h = RMSNorm(x) * weight                 (nn.RMSNorm, mamba_model.py:40,69)
// which the reference runs as separate MLX ops (two to four launches per layer in
// torch).  The row is read once, the sum of squares reduced in fp32, and both the
// updated residual and the normalised row written back -- HBM-bound at 3 x element
// size (+ 1 with the add) per element.
//
// Fast path (dim % 8 == 0, 16-byte aligned rows, dim <= 64 * 8 * kMaxChunks): one
// wave per row, 8-element vector loads and stores, a wave-only reduction (no LDS,
// no barrier), 4 rows per workgroup.  Anything else takes the generic kernel (one
// workgroup per row, element-wise).
#include "mm_common.h"

namespace mm {
namespace norm {

constexpr int kThreads = 256;
constexpr int kMaxPerThread = 32;  // dim <= 8192
constexpr int kMaxChunks = 8;      // fast path: dim <= 64 lanes x 8 chunks x 8 = 4096

template <int DT, int WT, bool ADD, int NCH>
__global__ __launch_bounds__(kThreads) void add_rmsnorm_vec_kernel(
    void* __restrict__ resid, const void* __restrict__ add, const void* __restrict__ weight,
    void* __restrict__ out, int64_t rows, int64_t dim, int64_t resid_stride, int64_t add_stride,
    int64_t out_stride, float eps) {
  using T = typename Ty<DT>::T;
  using TW = typename Ty<WT>::T;
  using V8 = typename Ty<DT>::V8;
  using W8 = typename Ty<WT>::V8;
  const int lane = threadIdx.x & 63;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * (kThreads / 64) + (threadIdx.x >> 6);
  if (row >= rows) return;  // whole wave: no barrier below
  T* r = static_cast<T*>(resid) + row * resid_stride;
  const T* a = static_cast<const T*>(add) + (ADD ? row * add_stride : 0);
  const int nch = static_cast<int>(dim >> 3);
  // All loads first, from clamped in-bounds chunks (chunk 0 past the row's end);
  // the values of those chunks are masked below.
  V8 rv[NCH], av[NCH];
  W8 wv[NCH];
#pragma unroll
  for (int i = 0; i < NCH; ++i) {
    const int ch = lane + 64 * i < nch ? lane + 64 * i : 0;
    rv[i] = *reinterpret_cast<const V8*>(r + 8 * ch);
    if constexpr (ADD) av[i] = *reinterpret_cast<const V8*>(a + 8 * ch);
    wv[i] = *reinterpret_cast<const W8*>(static_cast<const TW*>(weight) + 8 * ch);
  }
  float v[NCH][8];
  float ss = 0.0f;
#pragma unroll
  for (int i = 0; i < NCH; ++i) {
    const bool ok = lane + 64 * i < nch;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      float x = Ty<DT>::f(rv[i][k]);
      // residual stream kept in the activation dtype, as the reference's x + y
      if constexpr (ADD) x = Ty<DT>::f(Ty<DT>::from(x + Ty<DT>::f(av[i][k])));
      v[i][k] = ok ? x : 0.0f;
      ss = __builtin_fmaf(v[i][k], v[i][k], ss);
    }
    if constexpr (ADD) {
      if (ok) {
        V8 o;
#pragma unroll
        for (int k = 0; k < 8; ++k) o[k] = Ty<DT>::from(v[i][k]);
        *reinterpret_cast<V8*>(r + 8 * (lane + 64 * i)) = o;
      }
    }
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) ss += lane_xor(ss, off);
  const float inv = rsqrtf(ss / static_cast<float>(dim) + eps);
  T* o = static_cast<T*>(out) + row * out_stride;
#pragma unroll
  for (int i = 0; i < NCH; ++i) {
    if (lane + 64 * i < nch) {
      V8 ov;
#pragma unroll
      for (int k = 0; k < 8; ++k) ov[k] = norm_round<DT>(v[i][k], inv, Ty<WT>::f(wv[i][k]));
      *reinterpret_cast<V8*>(o + 8 * (lane + 64 * i)) = ov;
    }
  }
}

template <int DT>
__global__ __launch_bounds__(kThreads) void add_rmsnorm_kernel(
    void* __restrict__ resid, const void* __restrict__ add, const void* __restrict__ weight,
    void* __restrict__ out, int64_t dim, int64_t resid_stride, int64_t add_stride,
    int64_t out_stride, float eps, int32_t w_dtype) {
  using T = typename Ty<DT>::T;
  __shared__ float s_part[kThreads / 64];
  const int64_t row = blockIdx.x;
  const int tid = threadIdx.x;
  T* r = static_cast<T*>(resid) + row * resid_stride;
  const T* a = add ? static_cast<const T*>(add) + row * add_stride : nullptr;
  float v[kMaxPerThread];
  float ss = 0.0f;
#pragma unroll
  for (int i = 0; i < kMaxPerThread; ++i) {
    const int64_t c = tid + static_cast<int64_t>(i) * kThreads;
    float x = 0.0f;
    if (c < dim) {
      x = Ty<DT>::f(r[c]);
      if (a) {
        // residual stream kept in the activation dtype, as the reference's x + y
        const T s = Ty<DT>::from(x + Ty<DT>::f(a[c]));
        r[c] = s;
        x = Ty<DT>::f(s);
      }
    }
    v[i] = x;
    ss = __builtin_fmaf(x, x, ss);
  }
  // wave reduction, then across the 4 waves
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) ss += lane_xor(ss, off);
  if ((tid & 63) == 0) s_part[tid >> 6] = ss;
  __syncthreads();
  float tot = 0.0f;
#pragma unroll
  for (int w = 0; w < kThreads / 64; ++w) tot += s_part[w];
  const float inv = rsqrtf(tot / static_cast<float>(dim) + eps);
  T* o = static_cast<T*>(out) + row * out_stride;
#pragma unroll
  for (int i = 0; i < kMaxPerThread; ++i) {
    const int64_t c = tid + static_cast<int64_t>(i) * kThreads;
    if (c < dim) {
      const float w = w_dtype == MM_F32 ? ld<MM_F32>(weight, c)
                      : w_dtype == MM_F16 ? ld<MM_F16>(weight, c) : ld<MM_BF16>(weight, c);
      o[c] = norm_round<DT>(v[i], inv, w);
    }
  }
}

}  // namespace norm
}  // namespace mm

extern "C" {

int mm_add_rmsnorm(void* resid, const void* add, const void* weight, void* out, int64_t rows,
                   int64_t dim, int64_t resid_stride, int64_t add_stride, int64_t out_stride,
                   float eps, int32_t x_dtype, int32_t w_dtype, void* stream) {
  using namespace mm;
  using namespace mm::norm;
  clear_error();
  if (!resid || !weight || !out) return fail(MM_ERR_NULL_POINTER, "resid, weight and out are required");
  if (rows < 0 || dim < 0) return fail(MM_ERR_SHAPE, "negative size");
  if (dim > static_cast<int64_t>(kThreads) * kMaxPerThread)
    return fail(MM_ERR_SHAPE, "dim=%lld exceeds %d", (long long)dim, kThreads * kMaxPerThread);
  if (rows > 0x7fffffff) return fail(MM_ERR_SHAPE, "too many rows");
  if (!valid_dtype(x_dtype) || !valid_dtype(w_dtype)) return fail(MM_ERR_DTYPE, "bad dtype");
  if (!(eps >= 0.0f)) return fail(MM_ERR_SHAPE, "eps must be >= 0");
  if (rows == 0 || dim == 0) return MM_OK;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int64_t es = dtype_size(x_dtype), vb = 8 * es, wvb = 8 * dtype_size(w_dtype);
  const bool vec = dim % 8 == 0 && dim <= 64 * 8 * kMaxChunks && aligned(resid, vb) &&
                   aligned(out, vb) && aligned(weight, wvb) && (!add || aligned(add, vb)) &&
                   (resid_stride * es) % vb == 0 && (out_stride * es) % vb == 0 &&
                   (!add || (add_stride * es) % vb == 0);
  if (vec) {
    const dim3 vgrid(static_cast<unsigned>(ceil_div(rows, kThreads / 64)));
    const int64_t nch = dim / 8;
    const int nc = nch <= 128 ? 2 : nch <= 256 ? 4 : 8;  // chunks per lane
#define MM_NORMV(D, W, A, C)                                                                   \
  hipLaunchKernelGGL((add_rmsnorm_vec_kernel<D, W, A, C>), vgrid, dim3(kThreads), 0, s, resid, \
                     add, weight, out, rows, dim, resid_stride, add_stride, out_stride, eps)
#define MM_NORMV_C(D, W, A)                          \
  switch (nc) {                                      \
    case 2: MM_NORMV(D, W, A, 2); break;             \
    case 4: MM_NORMV(D, W, A, 4); break;             \
    default: MM_NORMV(D, W, A, 8); break;            \
  }
#define MM_NORMV_A(D, W)                             \
  if (add) {                                         \
    MM_NORMV_C(D, W, true)                           \
  } else {                                           \
    MM_NORMV_C(D, W, false)                          \
  }
#define MM_NORMV_W(D)                                \
  switch (w_dtype) {                                 \
    case MM_F32: MM_NORMV_A(D, MM_F32); break;       \
    case MM_F16: MM_NORMV_A(D, MM_F16); break;       \
    default: MM_NORMV_A(D, MM_BF16); break;          \
  }
    switch (x_dtype) {
      case MM_F32: MM_NORMV_W(MM_F32); break;
      case MM_F16: MM_NORMV_W(MM_F16); break;
      default: MM_NORMV_W(MM_BF16); break;
    }
#undef MM_NORMV_W
#undef MM_NORMV_A
#undef MM_NORMV_C
#undef MM_NORMV
    return check_launch("add_rmsnorm");
  }
  const dim3 grid(static_cast<unsigned>(rows));
#define MM_NORM(D)                                                                          \
  hipLaunchKernelGGL((add_rmsnorm_kernel<D>), grid, dim3(kThreads), 0, s, resid, add, weight, \
                     out, dim, resid_stride, add_stride, out_stride, eps, w_dtype)
  switch (x_dtype) {
    case MM_F32: MM_NORM(MM_F32); break;
    case MM_F16: MM_NORM(MM_F16); break;
    default: MM_NORM(MM_BF16); break;
  }
#undef MM_NORM
  return check_launch("add_rmsnorm");
}

}  // extern "C"
