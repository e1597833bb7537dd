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
        const float a = exp2_decay<DT>(dtl * as[k]);
        hs[k] = __builtin_fmaf(a, hs[k], du * ld<DT>(p.B, b * p.Bsb + n));
        acc = __builtin_fmaf(hs[k], ld<DT>(p.C, b * p.Csb + n), acc);
      }
      *reinterpret_cast<float4*>(hp + n4) = make_float4(hs[0], hs[1], hs[2], hs[3]);
    }
  } else {
#pragma unroll
    for (int n = 0; n < NS; ++n) {
      if (n < N) {
        const float a = exp2_decay<DT>(dtl * Ap[n]);
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

// ---------------------------------------------------------------------------
// Fused decode SSM step with the dt projection folded in: mm_decode_ssm_step_dtproj.
//
// Replaces mamba_block.py:183-195 INCLUDING the dt_proj Linear of :183:
//   dt[b,c] = softplus(bias[c] + sum_r dt_in[b,r] * W[c,r])
// followed by the state update of mm_decode_ssm_step (dstate == 16, the Mamba-1
// checkpoints' value).
//
// Lane layout: a channel's 16-float state row is split over a quad of 4
// consecutive lanes (4 states = one float4 each), so a wave covers 16 channels and
// every state access of a wave is 1 KB contiguous.  The rank-R dot product is
// split over the quad the same way: lane q holds W[c, q*RQ : (q+1)*RQ] in
// registers -- loaded once, reused for every batch row of the workgroup -- and
// reads the matching dt_in slice from LDS (padded so the quad's four broadcast
// reads hit distinct banks); two quad shuffles finish the dot and the C
// contraction.  All state rows of the workgroup are loaded before any compute so
// the kernel keeps kBB x 16 bytes per lane in flight: it is HBM-bound on the
// 2 x 64 bytes of state per (b, c).
namespace mm {
namespace dec {

constexpr int kFusedWaves = 2;
constexpr int kFusedCh = kFusedWaves * 16;   // channels per workgroup
constexpr int kFusedBB = 8;                  // batch rows per workgroup
constexpr int kFusedNS = 16;
constexpr int kMaxRank = 256;

struct FusedParams {
  float* h;
  const void* x;
  const void* dt_in;
  const void* w;
  const void* bias;
  const float* A;
  const void* B;
  const void* C;
  const float* D;
  const void* z;
  void* y;
  int64_t batch, dim, rank;
  int64_t xsb, dtsb, wsc, Bsb, Csb, zsb, ysb;
  int32_t wvec;  // W rows 16-byte aligned and rank % 8 == 0: 8-element vector loads
  int32_t mvec;  // also dt_in rows 16-byte aligned (2-byte types): matrix-core dt projection
};

// 8 consecutive elements at p (16-byte aligned for 2-byte types, 32 for fp32).
template <int DT>
__device__ __forceinline__ void ld8(const void* p, float* out) {
  using V8 = typename Ty<DT>::V8;
  const V8 v = *static_cast<const V8*>(p);
#pragma unroll
  for (int k = 0; k < 8; ++k) out[k] = Ty<DT>::f(v[k]);
}

template <int DT, int RQ, bool WVEC>
__global__ __launch_bounds__(kFusedWaves * 64) void ssm_step_dtproj_kernel(const FusedParams p) {
  using T = typename Ty<DT>::T;
  using V8 = typename Ty<DT>::V8;
  constexpr int RQP = RQ + 4;  // padded slice stride: quad reads land in distinct banks
  constexpr int NT = kFusedWaves * 64;
  __shared__ float s_dt[kFusedBB][4 * RQP];
  __shared__ float s_B[kFusedBB][kFusedNS];
  __shared__ float s_C[kFusedBB][kFusedNS];
  const int tid = threadIdx.x;
  const int q = tid & 3;
  const int64_t c = static_cast<int64_t>(blockIdx.x) * kFusedCh + (tid >> 2);
  const int64_t b0 = static_cast<int64_t>(blockIdx.y) * kFusedBB;
  const int nb = static_cast<int>(p.batch - b0 < kFusedBB ? p.batch - b0 : kFusedBB);
  const int R = static_cast<int>(p.rank);
  const bool cok = c < p.dim;
  // Every load below is unconditional from a clamped, in-bounds address (channel 0
  // past dim, row b0 past the batch, index 0 past rank); the values are masked at
  // their first use, so all loads are in flight together.
  const int64_t cc = cok ? c : 0;
  const T* const zp = static_cast<const T*>(p.z ? p.z : p.x);

  // Load order matters (the load counter is in order): dt_in rows, B and C first
  // (they gate the LDS staging and the barrier), then W, A, bias and D (needed by
  // every row), then the state rows: each row's update and store can start as soon
  // as its own state has arrived.
  constexpr int NDT = (kFusedBB * 4 * RQ + NT - 1) / NT;
  T dtr[NDT];
#pragma unroll
  for (int u = 0; u < NDT; ++u) {
    const int e = tid + u * NT;
    const int bb = e / (4 * RQ), r = e % (4 * RQ);
    const bool ok = e < kFusedBB * 4 * RQ && bb < nb && r < R;
    dtr[u] = static_cast<const T*>(p.dt_in)[ok ? (b0 + bb) * p.dtsb + r : 0];
  }
  constexpr int NBC = (kFusedBB * kFusedNS + NT - 1) / NT;
  T br[NBC], cr[NBC];
#pragma unroll
  for (int u = 0; u < NBC; ++u) {
    const int e = tid + u * NT;
    const int bb = e / kFusedNS, n = e % kFusedNS;
    const bool ok = e < kFusedBB * kFusedNS && bb < nb;
    br[u] = static_cast<const T*>(p.B)[ok ? (b0 + bb) * p.Bsb + n : 0];
    cr[u] = static_cast<const T*>(p.C)[ok ? (b0 + bb) * p.Csb + n : 0];
  }
  // This lane's slice of W[c, :] (zero beyond rank).
  const int r0 = q * RQ;
  float w[RQ];
  if constexpr (WVEC) {
    V8 raw[RQ / 8];
#pragma unroll
    for (int i = 0; i < RQ / 8; ++i) {
      const int r = r0 + 8 * i < R ? r0 + 8 * i : 0;
      raw[i] = *reinterpret_cast<const V8*>(static_cast<const T*>(p.w) + cc * p.wsc + r);
    }
#pragma unroll
    for (int i = 0; i < RQ / 8; ++i)
#pragma unroll
      for (int k = 0; k < 8; ++k) w[8 * i + k] = (r0 + 8 * i < R) ? Ty<DT>::f(raw[i][k]) : 0.0f;
  } else {
    T raw[RQ];
#pragma unroll
    for (int i = 0; i < RQ; ++i) {
      const int r = r0 + i < R ? r0 + i : 0;
      raw[i] = static_cast<const T*>(p.w)[cc * p.wsc + r];
    }
#pragma unroll
    for (int i = 0; i < RQ; ++i) w[i] = (r0 + i < R) ? Ty<DT>::f(raw[i]) : 0.0f;
  }
  float4 Av = *reinterpret_cast<const float4*>(p.A + cc * kFusedNS + q * 4);
  const T biasr = static_cast<const T*>(p.bias ? p.bias : p.x)[p.bias ? cc : 0];
  const float Dr = p.D ? p.D[cc] : 0.0f;
  float4 hv[kFusedBB];
  T xr[kFusedBB], zr[kFusedBB];
#pragma unroll
  for (int bb = 0; bb < kFusedBB; ++bb) {
    const int64_t b = b0 + (bb < nb ? bb : 0);
    hv[bb] = *reinterpret_cast<const float4*>(p.h + (b * p.dim + cc) * kFusedNS + q * 4);
    xr[bb] = static_cast<const T*>(p.x)[b * p.xsb + cc];
    zr[bb] = zp[p.z ? b * p.zsb + cc : b * p.xsb + cc];
  }

#pragma unroll
  for (int u = 0; u < NDT; ++u) {
    const int e = tid + u * NT;
    const int bb = e / (4 * RQ), r = e % (4 * RQ);
    if (e < kFusedBB * 4 * RQ)
      s_dt[bb][(r / RQ) * RQP + r % RQ] = (bb < nb && r < R) ? Ty<DT>::f(dtr[u]) : 0.0f;
  }
#pragma unroll
  for (int u = 0; u < NBC; ++u) {
    const int e = tid + u * NT;
    const int bb = e / kFusedNS, n = e % kFusedNS;
    if (e < kFusedBB * kFusedNS) {
      s_B[bb][n] = bb < nb ? Ty<DT>::f(br[u]) : 0.0f;
      s_C[bb][n] = bb < nb ? Ty<DT>::f(cr[u]) : 0.0f;
    }
  }
  __syncthreads();

  const float Al[4] = {Av.x * kLog2e, Av.y * kLog2e, Av.z * kLog2e, Av.w * kLog2e};
  const float bias = p.bias ? Ty<DT>::f(biasr) : 0.0f;
  float* hw = p.h + (b0 * p.dim + cc) * kFusedNS + q * 4;
#pragma unroll
  for (int bb = 0; bb < kFusedBB; ++bb) {
    if (bb >= nb) break;
    const float4* sd = reinterpret_cast<const float4*>(&s_dt[bb][q * RQP]);
    float dot = 0.0f;
#pragma unroll
    for (int i = 0; i < RQ / 4; ++i) {
      const float4 d = sd[i];
      dot = __builtin_fmaf(d.x, w[4 * i], dot);
      dot = __builtin_fmaf(d.y, w[4 * i + 1], dot);
      dot = __builtin_fmaf(d.z, w[4 * i + 2], dot);
      dot = __builtin_fmaf(d.w, w[4 * i + 3], dot);
    }
    dot += lane_xor(dot, 1);
    dot += lane_xor(dot, 2);
    const float xv = Ty<DT>::f(xr[bb]);
    const float dtv = softplus_full(dot + bias);
    const float du = dtv * xv;
    float hs[4] = {hv[bb].x, hv[bb].y, hv[bb].z, hv[bb].w};
    float acc = 0.0f;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const float a = exp2_decay<DT>(dtv * Al[k]);
      hs[k] = __builtin_fmaf(a, hs[k], du * s_B[bb][q * 4 + k]);
      acc = __builtin_fmaf(hs[k], s_C[bb][q * 4 + k], acc);
    }
    if (cok) *reinterpret_cast<float4*>(hw + bb * p.dim * kFusedNS) = make_float4(hs[0], hs[1], hs[2], hs[3]);
    acc += lane_xor(acc, 1);
    acc += lane_xor(acc, 2);
    if (q == 0 && cok) {
      acc = __builtin_fmaf(Dr, xv, acc);
      if (p.z) acc *= silu_f(Ty<DT>::f(zr[bb]));
      st<DT>(p.y, (b0 + bb) * p.ysb + c, acc);
    }
  }
}

// f16/bf16 variant with the dt projection on the matrix cores.  Workgroup = two waves =
// 32 channels x kMBB batch rows.  Wave w:
//   1. dt_pre[16 rows][16 channels] = dt_in[b0.., :] . W[c0 + 16w.., :]^T with KS
//      v_mfma_f32_16x16x32 steps (lane l: A = dt_in row l%16, B = W row l%16, k slice
//      8(l/16) .. +8 of each 32-wide step; C: rows 4(l/16) + i, column l%16);
//   2. the tile goes through a wave-private LDS block into the update layout:
//      lane l = channel l/4, states 4(l%4) .. +3, all kMBB rows;
//   3. the update of `ssm_step_dtproj_kernel` per row.
// All global loads are issued before the MFMAs (operands first, then the kMBB state
// rows, x and z), from clamped in-bounds addresses; masked values never reach a store.
// Batch rows per workgroup: 8 (measured faster than 16 on MI355X -- more, shorter
// workgroups overlap their state reads and writes better); the 16-row dt tile's
// upper half is computed and ignored.
constexpr int kMBB = 8;
static_assert(kMBB == 8 || kMBB == 16, "the dt tile has 16 rows");

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

template <int DT>
__device__ __forceinline__ f32x4 mfma16(u32x4 a, u32x4 b, f32x4 c) {
  if constexpr (DT == MM_F16)
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c,
                                                  0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b),
                                                   c, 0, 0, 0);
}

template <int DT, int KS>
__global__ __launch_bounds__(kFusedWaves * 64) void ssm_step_mfma_kernel(const FusedParams p) {
  using T = typename Ty<DT>::T;
  __shared__ float s_B[kMBB][kFusedNS];
  __shared__ float s_C[kMBB][kFusedNS];
  __shared__ float s_dt[kFusedWaves][16][17];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int64_t cw0 = static_cast<int64_t>(blockIdx.x) * kFusedCh + wave * 16;  // wave's channels
  const int64_t b0 = static_cast<int64_t>(blockIdx.y) * kMBB;
  const int R = static_cast<int>(p.rank);

  // ---- MFMA operands: dt_in row b0 + l%16, W row cw0 + l%16, k = 32 s + 8(l/16) ----
  const int64_t ar = b0 + (lane & 15) < p.batch ? b0 + (lane & 15) : 0;
  const int64_t wr = cw0 + (lane & 15) < p.dim ? cw0 + (lane & 15) : 0;
  const int kl = 8 * (lane >> 4);
  u32x4 av[KS], bv[KS];
#pragma unroll
  for (int s = 0; s < KS; ++s) {
    const int k = 32 * s + kl < R ? 32 * s + kl : 0;
    av[s] = *reinterpret_cast<const u32x4*>(static_cast<const T*>(p.dt_in) + ar * p.dtsb + k);
    bv[s] = *reinterpret_cast<const u32x4*>(static_cast<const T*>(p.w) + wr * p.wsc + k);
  }
  // ---- B / C rows of this workgroup (staged in LDS), then the per-lane update inputs ----
  constexpr int NBCU = kMBB * kFusedNS / (kFusedWaves * 64);
  T bcr[NBCU];
#pragma unroll
  for (int u = 0; u < NBCU; ++u) {
    const int e = tid + u * kFusedWaves * 64;  // rows x 16 states
    const int bb = e >> 4, n = e & 15;
    const int64_t row = b0 + bb < p.batch ? b0 + bb : 0;
    bcr[u] = static_cast<const T*>(p.B)[row * p.Bsb + n];
  }
  T ccr[NBCU];
#pragma unroll
  for (int u = 0; u < NBCU; ++u) {
    const int e = tid + u * kFusedWaves * 64;
    const int bb = e >> 4, n = e & 15;
    const int64_t row = b0 + bb < p.batch ? b0 + bb : 0;
    ccr[u] = static_cast<const T*>(p.C)[row * p.Csb + n];
  }
  const int q = lane & 3;
  const int cl = lane >> 2;
  const int64_t c = cw0 + cl;
  const bool cok = c < p.dim;
  const int64_t cc = cok ? c : 0;
  const float4 Av = *reinterpret_cast<const float4*>(p.A + cc * kFusedNS + q * 4);
  const T biasr = static_cast<const T*>(p.bias ? p.bias : p.x)[p.bias ? cc : 0];
  const float Dr = p.D ? p.D[cc] : 0.0f;
  const T* const zp = static_cast<const T*>(p.z ? p.z : p.x);
  f32x4 hv[kMBB];  // state rows: read and written once per step (non-temporal)
  T xr[kMBB], zr[kMBB];
#pragma unroll
  for (int bb = 0; bb < kMBB; ++bb) {
    const int64_t b = b0 + bb < p.batch ? b0 + bb : 0;
    hv[bb] = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(p.h + (b * p.dim + cc) * kFusedNS + q * 4));
    xr[bb] = static_cast<const T*>(p.x)[b * p.xsb + cc];
    zr[bb] = zp[p.z ? b * p.zsb + cc : b * p.xsb + cc];
  }

  // ---- dt_pre on the matrix cores (k past rank contributes zero) ----
  f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int s = 0; s < KS; ++s) {
    u32x4 a = av[s], w = bv[s];
    if (32 * s + kl >= R) a = u32x4{0u, 0u, 0u, 0u}, w = a;
    acc = mfma16<DT>(a, w, acc);
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) s_dt[wave][4 * (lane >> 4) + i][lane & 15] = acc[i];
#pragma unroll
  for (int u = 0; u < NBCU; ++u) {
    const int e = tid + u * kFusedWaves * 64;
    (&s_B[0][0])[e] = Ty<DT>::f(bcr[u]);
    (&s_C[0][0])[e] = Ty<DT>::f(ccr[u]);
  }
  __syncthreads();

  // ---- update: lane = (channel cl, states 4q .. 4q+3), rows b0 .. b0 + kMBB - 1 ----
  const float Al[4] = {Av.x * kLog2e, Av.y * kLog2e, Av.z * kLog2e, Av.w * kLog2e};
  const float bias = p.bias ? Ty<DT>::f(biasr) : 0.0f;
  float* const hw = p.h + (b0 * p.dim + cc) * kFusedNS + q * 4;
#pragma unroll
  for (int bb = 0; bb < kMBB; ++bb) {
    if (b0 + bb >= p.batch) break;
    const float xv = Ty<DT>::f(xr[bb]);
    const float dtv = softplus_full(s_dt[wave][bb][cl] + bias);
    const float du = dtv * xv;
    float hs[4] = {hv[bb][0], hv[bb][1], hv[bb][2], hv[bb][3]};
    float yacc = 0.0f;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const float a = exp2_decay<DT>(dtv * Al[k]);
      hs[k] = __builtin_fmaf(a, hs[k], du * s_B[bb][q * 4 + k]);
      yacc = __builtin_fmaf(hs[k], s_C[bb][q * 4 + k], yacc);
    }
    if (cok) __builtin_nontemporal_store(f32x4{hs[0], hs[1], hs[2], hs[3]}, reinterpret_cast<f32x4*>(hw + bb * p.dim * kFusedNS));
    yacc += lane_xor(yacc, 1);
    yacc += lane_xor(yacc, 2);
    if (q == 0 && cok) {
      yacc = __builtin_fmaf(Dr, xv, yacc);
      if (p.z) yacc *= silu_f(Ty<DT>::f(zr[bb]));
      st<DT>(p.y, (b0 + bb) * p.ysb + c, yacc);
    }
  }
}

template <int DT>
void launch_mfma(const FusedParams& p, hipStream_t s) {
  const dim3 grid(static_cast<unsigned>(ceil_div(p.dim, kFusedCh)),
                  static_cast<unsigned>(ceil_div(p.batch, kMBB)));
  const dim3 block(kFusedWaves * 64);
  switch (ceil_div(p.rank, 32)) {
    case 1: hipLaunchKernelGGL((ssm_step_mfma_kernel<DT, 1>), grid, block, 0, s, p); break;
    case 2: hipLaunchKernelGGL((ssm_step_mfma_kernel<DT, 2>), grid, block, 0, s, p); break;
    case 3: hipLaunchKernelGGL((ssm_step_mfma_kernel<DT, 3>), grid, block, 0, s, p); break;
    case 4: hipLaunchKernelGGL((ssm_step_mfma_kernel<DT, 4>), grid, block, 0, s, p); break;
    case 5: hipLaunchKernelGGL((ssm_step_mfma_kernel<DT, 5>), grid, block, 0, s, p); break;
    case 6: hipLaunchKernelGGL((ssm_step_mfma_kernel<DT, 6>), grid, block, 0, s, p); break;
    default: hipLaunchKernelGGL((ssm_step_mfma_kernel<DT, 8>), grid, block, 0, s, p); break;
  }
}

template <int DT, bool WV>
void launch_fused_w(const FusedParams& p, hipStream_t s) {
  const dim3 grid(static_cast<unsigned>(ceil_div(p.dim, kFusedCh)),
                  static_cast<unsigned>(ceil_div(p.batch, kFusedBB)));
  const dim3 block(kFusedWaves * 64);
  const int64_t rq = ceil_div(p.rank, 4);
  if (rq <= 16)
    hipLaunchKernelGGL((ssm_step_dtproj_kernel<DT, 16, WV>), grid, block, 0, s, p);
  else if (rq <= 32)
    hipLaunchKernelGGL((ssm_step_dtproj_kernel<DT, 32, WV>), grid, block, 0, s, p);
  else if (rq <= 48)
    hipLaunchKernelGGL((ssm_step_dtproj_kernel<DT, 48, WV>), grid, block, 0, s, p);
  else
    hipLaunchKernelGGL((ssm_step_dtproj_kernel<DT, 64, WV>), grid, block, 0, s, p);
}

template <int DT>
void launch_fused(const FusedParams& p, hipStream_t s) {
  if (DT != MM_F32 && p.mvec) launch_mfma<DT == MM_F32 ? MM_F16 : DT>(p, s);
  else if (p.wvec) launch_fused_w<DT, true>(p, s);
  else launch_fused_w<DT, false>(p, s);
}

}  // namespace dec
}  // namespace mm

extern "C" {

int mm_decode_ssm_step_dtproj(float* ssm_state, const void* x, const void* dt_in,
                              const void* dt_weight, const void* dt_bias, const float* A,
                              const void* B, const void* C, const float* D, const void* z,
                              void* y, int64_t batch, int64_t dim, int64_t dstate, int64_t rank,
                              int64_t x_stride_b, int64_t dt_stride_b, int64_t w_stride_c,
                              int64_t B_stride_b, int64_t C_stride_b, int64_t z_stride_b,
                              int64_t y_stride_b, int32_t x_dtype, int32_t w_dtype, void* stream) {
  using namespace mm;
  using namespace mm::dec;
  clear_error();
  if (!ssm_state || !x || !dt_in || !dt_weight || !A || !B || !C || !y)
    return fail(MM_ERR_NULL_POINTER, "ssm_state, x, dt_in, dt_weight, A, B, C and y are required");
  if (batch < 0 || dim < 0) return fail(MM_ERR_SHAPE, "negative size");
  if (rank < 1 || rank > kMaxRank)
    return fail(MM_ERR_SHAPE, "rank=%lld outside [1, %d]", (long long)rank, kMaxRank);
  if (dstate != kFusedNS)
    return fail(MM_ERR_DSTATE, "dstate=%lld: the fused step supports dstate == %d",
                (long long)dstate, kFusedNS);
  if (!valid_dtype(x_dtype) || !valid_dtype(w_dtype)) return fail(MM_ERR_DTYPE, "bad dtype");
  if (w_dtype != x_dtype)
    return fail(MM_ERR_DTYPE, "dt_weight dtype %d differs from x dtype %d", w_dtype, x_dtype);
  if (!aligned(ssm_state, 16) || !aligned(A, 16))
    return fail(MM_ERR_LAYOUT, "ssm_state and A must be 16-byte aligned");
  if (ceil_div(batch, kFusedBB) > 65535) return fail(MM_ERR_SHAPE, "batch too large");
  if (batch == 0 || dim == 0) return MM_OK;
  FusedParams p;
  p.h = ssm_state;
  p.x = x;
  p.dt_in = dt_in;
  p.w = dt_weight;
  p.bias = dt_bias;
  p.A = A;
  p.B = B;
  p.C = C;
  p.D = D;
  p.z = z;
  p.y = y;
  p.batch = batch;
  p.dim = dim;
  p.rank = rank;
  p.xsb = x_stride_b;
  p.dtsb = dt_stride_b;
  p.wsc = w_stride_c;
  p.Bsb = B_stride_b;
  p.Csb = C_stride_b;
  p.zsb = z_stride_b;
  p.ysb = y_stride_b;
  {
    const int64_t vb = x_dtype == MM_F32 ? 32 : 16;  // bytes of 8 elements
    const int64_t es = dtype_size(x_dtype);
    p.wvec = (rank % 8 == 0) && aligned(dt_weight, vb) && ((w_stride_c * es) % vb == 0) ? 1 : 0;
    p.mvec = (p.wvec && x_dtype != MM_F32 && aligned(dt_in, 16) && (dt_stride_b * es) % 16 == 0) ? 1 : 0;
  }
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (x_dtype) {
    case MM_F32: launch_fused<MM_F32>(p, s); break;
    case MM_F16: launch_fused<MM_F16>(p, s); break;
    default: launch_fused<MM_BF16>(p, s); break;
  }
  return check_launch("decode_ssm_step_dtproj");
}

}  // extern "C"
