// Causal depthwise conv1d (prefill) and the decode conv-window step.
//
// Prefill replaces MLX nn.Conv1d(groups=d_inner, padding=d_conv-1)[:, :L] + nn.silu
// (mamba_metal/mamba_block.py:45-52,77-78,129-130) and fuses the conv-state slice of
// mamba_block.py:118-127.  Each thread owns 8 adjacent channels (one 16-byte
// fp16 vector when channels are contiguous) and a run of TC timesteps; the
// (width-1)-deep causal window lives in registers and slides along time, so x
// is read once (plus a (width-1)-step halo per run) and out written once:
// HBM-bound at ~2 x element size bytes per (b, t, c).  The run is walked in groups
// of kU steps whose loads are all issued before any of them is used (clamped to the
// run's last step, so every load is in bounds and unconditional): one load in flight
// per thread left the kernel latency-bound at a third of the HBM rate.
//
// The decode step replaces mamba_block.py:170-177: shift the (batch, dim, width)
// window left in place, append x, dot with the taps, add bias, SiLU.
#include <algorithm>
#include <type_traits>

#include "mm_common.h"

namespace mm {
namespace conv {

constexpr int kCV = 8;      // channels per thread
constexpr int kU = 8;       // timesteps per load group
constexpr int kMaxW = 8;    // largest width accepted
constexpr int kBlock = 256;

struct Params {
  const void* x;
  const void* w;
  const void* bias;
  void* out;
  void* state;
  int64_t batch, seqlen, dim, width, tc, nchunks, ncg;
  int64_t xs0, xs1, xs2, os0, os1, os2, ws0, ws1;
  int32_t w_dtype, apply_silu, vec_ok;
  int32_t w_vec;  // 2-byte taps in contiguous rows of 4 (and bias) on 16-byte boundaries
};

__device__ __forceinline__ float ld_any(const void* p, int64_t i, int32_t dt) {
  return dt == MM_F32 ? ld<MM_F32>(p, i) : dt == MM_F16 ? ld<MM_F16>(p, i) : ld<MM_BF16>(p, i);
}

// K = compile-time width; K == 0 means "runtime width <= kMaxW" using a zero-padded
// kMaxW-tap window (taps aligned to the newest input).
template <int DT, int K, bool VEC>
__global__ __launch_bounds__(kBlock) void conv1d_kernel(const Params p) {
  using T = typename Ty<DT>::T;
  using V8 = typename Ty<DT>::V8;
  constexpr int W = K > 0 ? K : kMaxW;
  const int64_t gid = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x;
  const int64_t total = p.batch * p.nchunks * p.ncg;
  if (gid >= total) return;
  const int64_t cg = gid % p.ncg;
  const int64_t chunk = (gid / p.ncg) % p.nchunks;
  const int64_t b = gid / (p.ncg * p.nchunks);
  const int64_t c0 = cg * kCV;
  const int off = W - static_cast<int>(K > 0 ? K : p.width);  // leading zero taps (K == 0)

  // Taps (zero-padded at the old end when K == 0) and bias ((dim,) contiguous, w_dtype).
  // Every load is unconditional, from a clamped in-bounds address, and masked afterwards:
  // guarded loads compiled to one branch and one vmcnt(0) wait per tap (~40 dependent
  // round trips per thread, most of a short sequence's time).  The dtype dispatch is
  // hoisted out of the loops for the same reason.
  float w[kCV][W], bias[kCV];
  auto load_taps = [&](auto wdt) __attribute__((always_inline)) {
    constexpr int WDT = decltype(wdt)::value;
#pragma unroll
    for (int j = 0; j < kCV; ++j) {
      const int64_t c = c0 + j;
      const int64_t cc = c < p.dim ? c : 0;
#pragma unroll
      for (int k = 0; k < W; ++k) {
        const int kk = k - off;
        w[j][k] = ld<WDT>(p.w, cc * p.ws0 + (kk >= 0 ? kk : 0) * p.ws1);
      }
      bias[j] = ld<WDT>(p.bias != nullptr ? p.bias : p.w, p.bias != nullptr ? cc : 0);
    }
  };
  // Width 4 with 2-byte taps in contiguous (dim, 4) rows (the model's conv1d.weight): the
  // thread's 8 channels x 4 taps are 64 contiguous bytes, read as four 16-byte loads, and
  // its 8 biases as one.
  auto load_taps_vec = [&](auto wdt) __attribute__((always_inline)) {
    constexpr int WDT = decltype(wdt)::value;
    using WV = typename Ty<WDT>::V8;
    const int64_t cb = c0 < p.dim ? c0 : 0;
    const WV* const wv = reinterpret_cast<const WV*>(static_cast<const typename Ty<WDT>::T*>(p.w) + cb * 4);
    const WV r0 = wv[0], r1 = wv[1], r2 = wv[2], r3 = wv[3];
    const WV rb = *reinterpret_cast<const WV*>(static_cast<const typename Ty<WDT>::T*>(
        p.bias != nullptr ? p.bias : p.w) + (p.bias != nullptr ? cb : 0));
    const WV rr[4] = {r0, r1, r2, r3};
#pragma unroll
    for (int j = 0; j < kCV; ++j) {
#pragma unroll
      for (int k = 0; k < W; ++k) w[j][k] = Ty<WDT>::f(rr[(j * 4 + k) / 8][(j * 4 + k) % 8]);
      bias[j] = Ty<WDT>::f(rb[j]);
    }
  };
  bool taps_done = false;
  if constexpr (K == 4) {
    if (p.w_vec) {
      if (p.w_dtype == MM_F16) load_taps_vec(std::integral_constant<int, MM_F16>{});
      else load_taps_vec(std::integral_constant<int, MM_BF16>{});
      taps_done = true;
    }
  }
  if (!taps_done) {
    if (p.w_dtype == MM_F32) load_taps(std::integral_constant<int, MM_F32>{});
    else if (p.w_dtype == MM_F16) load_taps(std::integral_constant<int, MM_F16>{});
    else load_taps(std::integral_constant<int, MM_BF16>{});
  }
#pragma unroll
  for (int j = 0; j < kCV; ++j) {
    const bool cin = c0 + j < p.dim;
#pragma unroll
    for (int k = 0; k < W; ++k) w[j][k] = (cin && k >= off) ? w[j][k] : 0.0f;
    bias[j] = (cin && p.bias != nullptr) ? bias[j] : 0.0f;
  }

  // x[b, t, c0 .. c0 + 7] (t >= 0); channels past dim read as zero.
  // Unconditional loads here too: on the vector path every thread's channel group lies
  // inside dim (dim % 8 == 0); the strided path reads channel 0 past dim and masks.
  auto load_x = [&](int64_t t, float v[kCV]) {
    const T* xp = static_cast<const T*>(p.x) + b * p.xs0 + t * p.xs1;
    if constexpr (VEC) {
      const V8 r = *reinterpret_cast<const V8*>(xp + c0);
#pragma unroll
      for (int j = 0; j < kCV; ++j) v[j] = Ty<DT>::f(r[j]);
    } else {
      float raw[kCV];
#pragma unroll
      for (int j = 0; j < kCV; ++j) raw[j] = Ty<DT>::f(xp[(c0 + j < p.dim ? c0 + j : 0) * p.xs2]);
#pragma unroll
      for (int j = 0; j < kCV; ++j) v[j] = (c0 + j < p.dim) ? raw[j] : 0.0f;
    }
  };

  const int64_t t_begin = chunk * p.tc;
  const int64_t t_end = std::min<int64_t>(t_begin + p.tc, p.seqlen);

  // win[k] holds x[t - (W-1) + k] for k < W-1 (the causal history): loaded from step 0
  // where t < 0 (unconditional loads, see the taps) and zeroed after.
  float win[W > 1 ? W - 1 : 1][kCV];
#pragma unroll
  for (int k = 0; k < W - 1; ++k) {
    const int64_t t = t_begin - (W - 1) + k;
    load_x(t >= 0 ? t : 0, win[k]);
  }
#pragma unroll
  for (int k = 0; k < W - 1; ++k) {
    const bool tin = t_begin - (W - 1) + k >= 0;
#pragma unroll
    for (int j = 0; j < kCV; ++j) win[k][j] = tin ? win[k][j] : 0.0f;
  }

  // Vector path: the group's raw 16-byte rows are loaded before any is converted (every
  // thread's channel group is inside dim there, so no load is guarded).
  constexpr int U = VEC ? kU : 1;
  const T* const xb = static_cast<const T*>(p.x) + b * p.xs0 + c0;
  for (int64_t t0 = t_begin; t0 < t_end; t0 += U) {
  V8 xr[U];
  float xs[VEC ? 1 : kCV];
  if constexpr (VEC) {
#pragma unroll
    for (int u = 0; u < U; ++u)
      xr[u] = *reinterpret_cast<const V8*>(xb + (t0 + u < t_end ? t0 + u : t_end - 1) * p.xs1);
  } else {
    load_x(t0, xs);
  }
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int64_t t = t0 + u;
    if (t >= t_end) break;
    float xn[kCV];
#pragma unroll
    for (int j = 0; j < kCV; ++j) {
      if constexpr (VEC) xn[j] = Ty<DT>::f(xr[u][j]);
      else xn[j] = xs[j];
    }
    float o[kCV];
#pragma unroll
    for (int j = 0; j < kCV; ++j) {
      float acc = bias[j];
#pragma unroll
      for (int k = 0; k < W - 1; ++k) acc = __builtin_fmaf(w[j][k], win[k][j], acc);
      acc = __builtin_fmaf(w[j][W - 1], xn[j], acc);
      o[j] = p.apply_silu ? silu_f(acc) : acc;
    }
    T* op = static_cast<T*>(p.out) + b * p.os0 + t * p.os1;
    if constexpr (VEC) {
      if (c0 < p.dim) {
        V8 r;
#pragma unroll
        for (int j = 0; j < kCV; ++j) r[j] = Ty<DT>::from(o[j]);
        *reinterpret_cast<V8*>(op + c0) = r;
      }
    } else {
#pragma unroll
      for (int j = 0; j < kCV; ++j)
        if (c0 + j < p.dim) op[(c0 + j) * p.os2] = Ty<DT>::from(o[j]);
    }
    // conv_state_out[b, c, kk] = x[seqlen - width + kk] (mamba_block.py:118-127):
    // at the last step the window win[0..W-2] ++ xn holds x[t-(W-1) .. t], zeros
    // where the index is negative.
    if (p.state != nullptr && t == p.seqlen - 1) {
      const int width = static_cast<int>(p.width);
#pragma unroll
      for (int j = 0; j < kCV; ++j) {
        const int64_t c = c0 + j;
        if (c >= p.dim) continue;
        T* sp = static_cast<T*>(p.state) + (b * p.dim + c) * width;
#pragma unroll
        for (int k = 0; k < W; ++k) {
          const int kk = k - (W - width);
          if (kk >= 0) sp[kk] = Ty<DT>::from(k == W - 1 ? xn[j] : win[k][j]);
        }
      }
    }
#pragma unroll
    for (int k = 0; k + 1 < W - 1; ++k)
#pragma unroll
      for (int j = 0; j < kCV; ++j) win[k][j] = win[k + 1][j];
    if (W > 1) {
#pragma unroll
      for (int j = 0; j < kCV; ++j) win[W - 2][j] = xn[j];
    }
  }
  }
}

template <int DT>
void launch_dt(const Params& p, hipStream_t s) {
  const int64_t total = p.batch * p.nchunks * p.ncg;
  const dim3 grid(static_cast<unsigned>(ceil_div(total, kBlock)));
#define MM_CONV_W(V)                                                                          \
  switch (p.width) {                                                                          \
    case 2: hipLaunchKernelGGL((conv1d_kernel<DT, 2, V>), grid, dim3(kBlock), 0, s, p); break; \
    case 3: hipLaunchKernelGGL((conv1d_kernel<DT, 3, V>), grid, dim3(kBlock), 0, s, p); break; \
    case 4: hipLaunchKernelGGL((conv1d_kernel<DT, 4, V>), grid, dim3(kBlock), 0, s, p); break; \
    default: hipLaunchKernelGGL((conv1d_kernel<DT, 0, V>), grid, dim3(kBlock), 0, s, p); break; \
  }
  if (p.vec_ok) {
    MM_CONV_W(true)
  } else {
    MM_CONV_W(false)
  }
#undef MM_CONV_W
}

// ---------------------------------------------------------------------------
// Decode conv-window step: one thread per (b, c).
struct StepParams {
  void* state;
  const void* x;
  const void* w;
  const void* bias;
  void* out;
  int64_t batch, dim, width, xsb, osb, ws0, ws1;
  int32_t s_dtype, x_dtype, w_dtype, apply_silu;
};

__device__ __forceinline__ void st_any(void* p, int64_t i, float v, int32_t dt) {
  if (dt == MM_F32)
    st<MM_F32>(p, i, v);
  else if (dt == MM_F16)
    st<MM_F16>(p, i, v);
  else
    st<MM_BF16>(p, i, v);
}

__global__ __launch_bounds__(kBlock) void conv_step_kernel(const StepParams p) {
  const int64_t c = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x;
  const int64_t b = blockIdx.y;
  if (c >= p.dim) return;
  const int width = static_cast<int>(p.width);
  const int64_t sbase = (b * p.dim + c) * p.width;
  float win[kMaxW];
#pragma unroll
  for (int k = 0; k < kMaxW; ++k)
    win[k] = (k + 1 < width) ? ld_any(p.state, sbase + k + 1, p.s_dtype) : 0.0f;
  const float xv = ld_any(p.x, b * p.xsb + c, p.x_dtype);
  float acc = p.bias ? ld_any(p.bias, c, p.w_dtype) : 0.0f;
#pragma unroll
  for (int k = 0; k < kMaxW; ++k) {
    if (k < width) {
      const float v = (k == width - 1) ? xv : win[k];
      acc = __builtin_fmaf(ld_any(p.w, c * p.ws0 + k * p.ws1, p.w_dtype), v, acc);
      st_any(p.state, sbase + k, v, p.s_dtype);
    }
  }
  st_any(p.out, b * p.osb + c, p.apply_silu ? silu_f(acc) : acc, p.x_dtype);
}

// Fast decode step for the common layout: width 4, state, x and weight of one
// dtype, state rows and weight rows contiguous and aligned.  The 4-tap window and
// the weight row move as single 8/16-byte vectors; the shifted window is written
// back with one vector store.
template <int DT>
__global__ __launch_bounds__(kBlock) void conv_step4_kernel(const StepParams p) {
  using T = typename Ty<DT>::T;
  typedef T T4 __attribute__((ext_vector_type(4)));
  const int64_t c = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x;
  const int64_t b = blockIdx.y;
  if (c >= p.dim) return;
  T4* sp = static_cast<T4*>(p.state) + b * p.dim + c;
  const T4 win = *sp;
  const T4 wv = static_cast<const T4*>(p.w)[c];
  const T xr = static_cast<const T*>(p.x)[b * p.xsb + c];
  float acc = p.bias ? ld<DT>(p.bias, c) : 0.0f;
  acc = __builtin_fmaf(Ty<DT>::f(wv[0]), Ty<DT>::f(win[1]), acc);
  acc = __builtin_fmaf(Ty<DT>::f(wv[1]), Ty<DT>::f(win[2]), acc);
  acc = __builtin_fmaf(Ty<DT>::f(wv[2]), Ty<DT>::f(win[3]), acc);
  acc = __builtin_fmaf(Ty<DT>::f(wv[3]), Ty<DT>::f(xr), acc);
  T4 nw;
  nw[0] = win[1];
  nw[1] = win[2];
  nw[2] = win[3];
  nw[3] = xr;
  *sp = nw;
  st<DT>(p.out, b * p.osb + c, p.apply_silu ? silu_f(acc) : acc);
}

}  // namespace conv
}  // namespace mm

extern "C" {

int mm_causal_conv1d_fwd(const void* x, const void* weight, const void* bias, void* out,
                         void* conv_state_out, int64_t batch, int64_t seqlen, int64_t dim,
                         int64_t width, const int64_t x_stride[3], const int64_t out_stride[3],
                         const int64_t w_stride[2], int32_t x_dtype, int32_t w_dtype,
                         int32_t apply_silu, void* stream) {
  using namespace mm;
  using namespace mm::conv;
  clear_error();
  if (!x || !weight || !out || !x_stride || !out_stride || !w_stride)
    return fail(MM_ERR_NULL_POINTER, "x, weight, out and the stride arrays are required");
  if (batch < 0 || seqlen < 0 || dim < 0)
    return fail(MM_ERR_SHAPE, "negative size (batch=%lld seqlen=%lld dim=%lld)",
                (long long)batch, (long long)seqlen, (long long)dim);
  if (width < 1 || width > kMaxW)
    return fail(MM_ERR_SHAPE, "width=%lld outside [1, %d]", (long long)width, kMaxW);
  if (!valid_dtype(x_dtype) || !valid_dtype(w_dtype))
    return fail(MM_ERR_DTYPE, "bad dtype (x_dtype=%d w_dtype=%d)", x_dtype, w_dtype);
  if (batch == 0 || seqlen == 0 || dim == 0) return MM_OK;

  Params p;
  p.x = x;
  p.w = weight;
  p.bias = bias;
  p.out = out;
  p.state = conv_state_out;
  p.batch = batch;
  p.seqlen = seqlen;
  p.dim = dim;
  p.width = width;
  p.xs0 = x_stride[0]; p.xs1 = x_stride[1]; p.xs2 = x_stride[2];
  p.os0 = out_stride[0]; p.os1 = out_stride[1]; p.os2 = out_stride[2];
  p.ws0 = w_stride[0];
  p.ws1 = w_stride[1];
  p.w_dtype = w_dtype;
  p.apply_silu = apply_silu ? 1 : 0;
  const int64_t vb = kCV * dtype_size(x_dtype);
  p.vec_ok = (p.xs2 == 1 && p.os2 == 1 && dim % kCV == 0 && aligned(x, vb) && aligned(out, vb) &&
              p.xs0 % kCV == 0 && p.xs1 % kCV == 0 && p.os0 % kCV == 0 && p.os1 % kCV == 0)
                 ? 1
                 : 0;
  p.ncg = ceil_div(dim, kCV);
  p.w_vec = (width == 4 && w_dtype != MM_F32 && p.ws1 == 1 && p.ws0 == 4 && dim % kCV == 0 &&
             aligned(weight, 16) && (bias == nullptr || aligned(bias, 16)))
                ? 1
                : 0;
  // Run length: enough runs for >= ~256k threads (~16 waves per CU), runs of at most
  // 256 steps and at least kU (one load group; the (width-1)-step halo is re-read per run).
  int64_t tc = 256;
  while (tc > kU && batch * p.ncg * ceil_div(seqlen, tc) < 262144) tc /= 2;
  p.tc = tc;
  p.nchunks = ceil_div(seqlen, tc);

  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (x_dtype) {
    case MM_F32: launch_dt<MM_F32>(p, s); break;
    case MM_F16: launch_dt<MM_F16>(p, s); break;
    default: launch_dt<MM_BF16>(p, s); break;
  }
  return check_launch("causal_conv1d");
}

int mm_decode_conv_step(void* conv_state, const void* x, const void* weight, const void* bias,
                        void* out, int64_t batch, int64_t dim, int64_t width,
                        int64_t x_stride_b, int64_t out_stride_b, const int64_t w_stride[2],
                        int32_t state_dtype, int32_t x_dtype, int32_t w_dtype,
                        int32_t apply_silu, void* stream) {
  using namespace mm;
  using namespace mm::conv;
  clear_error();
  if (!conv_state || !x || !weight || !out || !w_stride)
    return fail(MM_ERR_NULL_POINTER, "conv_state, x, weight, out and w_stride are required");
  if (batch < 0 || dim < 0) return fail(MM_ERR_SHAPE, "negative size");
  if (width < 1 || width > kMaxW)
    return fail(MM_ERR_SHAPE, "width=%lld outside [1, %d]", (long long)width, kMaxW);
  if (batch > 65535) return fail(MM_ERR_SHAPE, "batch=%lld exceeds 65535", (long long)batch);
  if (!valid_dtype(state_dtype) || !valid_dtype(x_dtype) || !valid_dtype(w_dtype))
    return fail(MM_ERR_DTYPE, "bad dtype");
  if (batch == 0 || dim == 0) return MM_OK;
  StepParams p;
  p.state = conv_state;
  p.x = x;
  p.w = weight;
  p.bias = bias;
  p.out = out;
  p.batch = batch;
  p.dim = dim;
  p.width = width;
  p.xsb = x_stride_b;
  p.osb = out_stride_b;
  p.ws0 = w_stride[0];
  p.ws1 = w_stride[1];
  p.s_dtype = state_dtype;
  p.x_dtype = x_dtype;
  p.w_dtype = w_dtype;
  p.apply_silu = apply_silu ? 1 : 0;
  const dim3 grid(static_cast<unsigned>(ceil_div(dim, kBlock)), static_cast<unsigned>(batch));
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int64_t vb = 4 * dtype_size(x_dtype);
  const bool fast = width == 4 && state_dtype == x_dtype && w_dtype == x_dtype &&
                    w_stride[1] == 1 && w_stride[0] == 4 && aligned(conv_state, vb) &&
                    aligned(weight, vb);
  if (fast) {
    switch (x_dtype) {
      case MM_F32: hipLaunchKernelGGL((conv_step4_kernel<MM_F32>), grid, dim3(kBlock), 0, s, p); break;
      case MM_F16: hipLaunchKernelGGL((conv_step4_kernel<MM_F16>), grid, dim3(kBlock), 0, s, p); break;
      default: hipLaunchKernelGGL((conv_step4_kernel<MM_BF16>), grid, dim3(kBlock), 0, s, p); break;
    }
  } else {
    hipLaunchKernelGGL(conv_step_kernel, grid, dim3(kBlock), 0, s, p);
  }
  return check_launch("decode_conv_step");
}

}  // extern "C"
