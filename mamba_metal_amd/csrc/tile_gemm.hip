// Prefill projection GEMM with short K: mm_prefill_linear.
//
// Replaces the dt projection of the parallel prefill (MambaBlock.prefill: dt_proj with its
// bias, mamba_metal/mamba_block.py:136), K = dt_rank:
//   y[m, n] = round(sum_k x[m, k] * w[n, k] (+ bias[n])),   fp32 accumulation.
// With so short a K the product is bound by its output stream and by launch-to-store
// latency, and a library GEMM's LDS pipeline is overhead.  Both operands are K-contiguous
// -- x rows (here the strided dt slice of x_proj's output) and the rows of nn.Linear's
// (N, K) weight -- which is the matrix cores' operand layout: for v_mfma_f32_32x32x16,
// lane l takes the 8 consecutive k of row (or weight row) l % 32 starting at 8 (l / 32).
// Every operand is one 16-byte global load per lane and step, straight into registers.
// The kernel takes any K that is a multiple of 16, but for deep products (the other
// projections) it runs L1-bound (operands are not shared through LDS) and the library
// GEMM is faster; the host routes only short K here.
//
// Workgroup = 4 waves.  Wave w takes K slice w % KS and output block w / KS of a WM x WN
// arrangement; a block is TM x TN tiles of 32 x 32.  Steps are loaded in groups of kU,
// two groups in flight (the next group's loads are issued before this group's MFMAs).
// With KS > 1 the waves of a block leave their fp32 partial tiles in LDS and the first
// sums them in slice order (a fixed order: results are reproducible).  Loads are
// unconditional from clamped, in-bounds addresses (rows past M read row 0, columns
// past N weight row 0, steps past a slice its last step); clamped rows and columns only
// feed outputs that are never stored, clamped steps are never multiplied in.
#include "mm_common.h"

namespace mm {
namespace tile {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

constexpr int kStep = 16;  // k per MFMA
constexpr int kU = 2;      // steps per load group

struct Params {
  const void* x;
  const void* w;
  const void* bias;
  void* y;
  int64_t M, N, K, ldx, ldw, ldy;
};

template <int DT>
__device__ __forceinline__ f32x16 mfma(u32x4 a, u32x4 b, f32x16 c) {
  if constexpr (DT == MM_F16)
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}

// Output layout of a 32x32 tile: lane l, register i holds row 8 (i / 4) + 4 (l / 32) +
// i % 4, column l % 32.
__device__ __forceinline__ int acc_row(int i, int lane) { return 8 * (i >> 2) + 4 * (lane >> 5) + (i & 3); }

template <int DT, int TM, int TN, int WM, int WN, int KS, bool BIAS>
__global__ __launch_bounds__(256) void tile_kernel(const Params p) {
  static_assert(WM * WN * KS == 4, "four waves per workgroup");
  using T = typename Ty<DT>::T;
  constexpr int NB = TM * TN * 16;  // accumulator floats per lane
  __shared__ float s_red[KS > 1 ? 4 : 1][KS > 1 ? NB : 1][64];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int ks = wave % KS;
  const int blk = wave / KS;
  const int wm = blk / WN, wn = blk % WN;
  const int64_t m0 = static_cast<int64_t>(blockIdx.y) * (32 * TM * WM) + wm * 32 * TM;
  const int64_t n0 = static_cast<int64_t>(blockIdx.x) * (32 * TN * WN) + wn * 32 * TN;
  const int64_t nsteps = p.K / kStep;
  const int64_t per = (nsteps + KS - 1) / KS;
  const int64_t s_begin = ks * per;
  const int64_t s_end = s_begin + per < nsteps ? s_begin + per : nsteps;

  const T* xr[TM];
  const T* wr[TN];
#pragma unroll
  for (int i = 0; i < TM; ++i) {
    const int64_t r = m0 + 32 * i + (lane & 31);
    xr[i] = static_cast<const T*>(p.x) + (r < p.M ? r : 0) * p.ldx + 8 * (lane >> 5);
  }
#pragma unroll
  for (int j = 0; j < TN; ++j) {
    const int64_t c = n0 + 32 * j + (lane & 31);
    wr[j] = static_cast<const T*>(p.w) + (c < p.N ? c : 0) * p.ldw + 8 * (lane >> 5);
  }
  float bv[TN];
#pragma unroll
  for (int j = 0; j < TN; ++j) {
    const int64_t c = n0 + 32 * j + (lane & 31);
    bv[j] = BIAS ? Ty<DT>::f(static_cast<const T*>(p.bias)[c < p.N ? c : 0]) : 0.0f;
  }

  f32x16 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

  if (s_begin < s_end) {
    const int64_t s_last = s_end - 1;
    u32x4 xa[kU][TM], wa[kU][TN], xb[kU][TM], wb[kU][TN];
    auto load = [&](u32x4(&xv)[kU][TM], u32x4(&wv)[kU][TN], int64_t s0) __attribute__((always_inline)) {
#pragma unroll
      for (int u = 0; u < kU; ++u) {
        const int64_t s = s0 + u <= s_last ? s0 + u : s_last;
#pragma unroll
        for (int i = 0; i < TM; ++i) xv[u][i] = *reinterpret_cast<const u32x4*>(xr[i] + s * kStep);
#pragma unroll
        for (int j = 0; j < TN; ++j) wv[u][j] = *reinterpret_cast<const u32x4*>(wr[j] + s * kStep);
      }
    };
    auto compute = [&](const u32x4(&xv)[kU][TM], const u32x4(&wv)[kU][TN], int64_t s0)
                       __attribute__((always_inline)) {
#pragma unroll
      for (int u = 0; u < kU; ++u) {
        if (s0 + u >= s_end) break;  // wave-uniform
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
          for (int j = 0; j < TN; ++j) acc[i][j] = mfma<DT>(xv[u][i], wv[u][j], acc[i][j]);
      }
    };
    load(xa, wa, s_begin);
    for (int64_t s = s_begin; s < s_end; s += 2 * kU) {
      load(xb, wb, s + kU);
      compute(xa, wa, s);
      load(xa, wa, s + 2 * kU);
      compute(xb, wb, s + kU);
    }
  }

  if constexpr (KS > 1) {
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) s_red[wave][(i * TN + j) * 16 + r][lane] = acc[i][j][r];
    __syncthreads();
    if (ks != 0) return;
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          float v = s_red[wave][(i * TN + j) * 16 + r][lane];
#pragma unroll
          for (int k = 1; k < KS; ++k) v += s_red[wave + k][(i * TN + j) * 16 + r][lane];
          acc[i][j][r] = v;
        }
  }

#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int64_t n = n0 + 32 * j + (lane & 31);
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int64_t m = m0 + 32 * i + acc_row(r, lane);
        if (m < p.M && n < p.N) st<DT>(p.y, m * p.ldy + n, acc[i][j][r] + bv[j]);
      }
    }
}

// Launch shapes: 64 x 64 workgroup tiles (2 x 2 waves of one 32 x 32 tile), or for
// narrow outputs (N <= 96) 32 x 32 blocks with K split over the four waves.  Measured on
// MI355X at the Mamba-130M prefill's dt_proj (2048 x 1536, K = 48 + bias): 5.7 us against
// 9.1 us for the library GEMM; 64 x 128 tiles 5.9 us.
struct Shape {
  int tm, tn, wm, wn, ks;
};

inline Shape pick(int64_t N) {
  if (N <= 96) return Shape{1, 1, 1, 1, 4};
  return Shape{1, 1, 2, 2, 1};
}

template <int DT, int TM, int TN, int WM, int WN, int KS>
void launch_t(const Params& p, bool bias, hipStream_t s) {
  const dim3 grid(static_cast<unsigned>(ceil_div(p.N, 32 * TN * WN)),
                  static_cast<unsigned>(ceil_div(p.M, 32 * TM * WM)));
  if (bias)
    hipLaunchKernelGGL((tile_kernel<DT, TM, TN, WM, WN, KS, true>), grid, dim3(256), 0, s, p);
  else
    hipLaunchKernelGGL((tile_kernel<DT, TM, TN, WM, WN, KS, false>), grid, dim3(256), 0, s, p);
}

template <int DT>
void launch(const Params& p, const Shape& sh, hipStream_t s) {
  const bool b = p.bias != nullptr;
  if (sh.ks == 4) launch_t<DT, 1, 1, 1, 1, 4>(p, b, s);
  else launch_t<DT, 1, 1, 2, 2, 1>(p, b, s);
}

inline int64_t max_grid_y(const Shape& s) { return 65535LL * 32 * s.tm * s.wm; }

}  // namespace tile
}  // namespace mm

extern "C" {

int mm_prefill_linear(const void* x, const void* w, const void* bias, void* y, int64_t M,
                      int64_t N, int64_t K, int64_t ldx, int64_t ldw, int64_t ldy, int32_t dtype,
                      void* stream) {
  using namespace mm;
  using namespace mm::tile;
  clear_error();
  if (!x || !w || !y) return fail(MM_ERR_NULL_POINTER, "x, w and y are required");
  if (dtype != MM_F16 && dtype != MM_BF16) return fail(MM_ERR_DTYPE, "dtype %d: f16 or bf16 only", dtype);
  if (M < 0 || N < 0 || K < 0) return fail(MM_ERR_SHAPE, "negative size");
  if (K % kStep != 0) return fail(MM_ERR_SHAPE, "K=%lld is not a multiple of %d", (long long)K, kStep);
  if (ldx < K || ldw < K || ldy < N) return fail(MM_ERR_LAYOUT, "row stride smaller than the row");
  if (ldx % 8 != 0 || ldw % 8 != 0)
    return fail(MM_ERR_LAYOUT, "ldx and ldw must be multiples of 8 elements (16-byte rows)");
  if (!aligned(x, 16) || !aligned(w, 16)) return fail(MM_ERR_LAYOUT, "x and w must be 16-byte aligned");
  if (M == 0 || N == 0) return MM_OK;
  const Shape sh = pick(N);
  if (M > max_grid_y(sh) || ceil_div(N, 32) > 0x7fffffffLL) return fail(MM_ERR_SHAPE, "too large");
  Params p;
  p.x = x;
  p.w = w;
  p.bias = bias;
  p.y = y;
  p.M = M;
  p.N = N;
  p.K = K;
  p.ldx = ldx;
  p.ldw = ldw;
  p.ldy = ldy;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (dtype == MM_F16) launch<MM_F16>(p, sh, s);
  else launch<MM_BF16>(p, sh, s);
  return check_launch("prefill_linear");
}

}  // extern "C"
