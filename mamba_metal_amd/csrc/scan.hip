// Chunked selective scan for gfx950 (MI355X): mm_selective_scan_fwd[_strided].
//
// Semantics follow mamba_metal/kernels/selective_scan_chunked.metal:28-155
// (softplus cutoff :60-65, discretisation :78-79, y accumulation :126-128,
// SiLU(z) gate :140-144, final state :151-155) and the op wrapper
// mamba_metal/selective_scan.py:23-80.  The decomposition is this library's own:
//
//   * One workgroup = 64 channels (one per lane) of one batch row x 4 state
//     groups (one per wave).  Each lane walks time SEQUENTIALLY and keeps its
//     SPL = ceil(dstate/4) states in fp32 registers, so the recurrence costs
//     exactly one exp2 + four VALU ops per (channel, state, step) and there is
//     no parallel-scan overhead at all: parallelism comes from the
//     batch*dim*4 independent (channel, state-group) recurrences.
//   * B and C are identical for every channel of a batch row.  A tiny pack
//     kernel rewrites them once into fp32 [batch][group][time][B(SPL),C(SPL)]
//     in the workspace, so inside the scan loop they are wave-uniform
//     addresses: the compiler fetches them with s_load into SGPRs and the
//     VALU reads them as scalar operands (no LDS, no VGPRs, no per-lane loads).
//   * Per time tile (32 steps) the whole workgroup runs a prologue over the
//     64x32 (channel, time) elements -- coalesced 16-byte loads of u, delta, z
//     along whichever axis is contiguous, softplus, delta*u, D*u, SiLU(z) --
//     and stores delta' and delta'*u to LDS; the 4 waves then scan; then the
//     epilogue sums the 4 per-group partial y from LDS, adds D*u, applies the
//     gate and stores y with 16-byte stores.  The next tile's raw loads are
//     issued before the scan so HBM latency hides under the VALU work.
//   * The running state never leaves registers between tiles (the reference
//     keeps a threadgroup-memory carry, selective_scan_chunked.metal:37-47).
#include "mm_common.h"

namespace mm {
namespace scan {

constexpr int kCPW = 64;                 // channels per workgroup (lanes per wave)
constexpr int kGroups = 4;               // state groups = waves per workgroup
constexpr int kThreads = kCPW * kGroups; // 256
constexpr int kT = 32;                   // timesteps per tile
constexpr int kTP = kT + 4;              // padded LDS row length (floats)
constexpr int kVec = 8;                  // elements per prologue/epilogue vector
static_assert(kCPW * kT / kVec == kThreads, "one vector per thread per tile");

enum Layout { kTimeContig = 0, kChanContig = 1 };

struct Params {
  const void* u;
  const void* delta;
  const void* z;
  void* y;
  const float* A;
  const float* D;
  float* state_out;
  const float* bc;  // packed B/C
  int64_t dim, dstate, seqlen, Lp, ntiles;
  int64_t us0, us1, us2, ds0, ds1, ds2, zs0, zs1, zs2, ys0, ys1, ys2;
  int64_t As0, As1, Ds;
  int32_t softplus;
  int32_t vec_ok;
};

inline int spl_for(int64_t dstate) {
  return dstate <= 4 ? 1 : dstate <= 8 ? 2 : dstate <= 16 ? 4 : dstate <= 32 ? 8 : 16;
}

// ---------------------------------------------------------------------------
// B/C pack: bc[((b*4 + g)*Lp + t)*2*SPL + k]       = B[b, g*SPL + k, t]
//           bc[((b*4 + g)*Lp + t)*2*SPL + SPL + k] = C[b, g*SPL + k, t]
// zero for padded states (n >= dstate) and padded steps (t >= seqlen).
template <int DT, int SPL>
__global__ __launch_bounds__(256) void pack_bc_kernel(const void* __restrict__ B,
                                                      const void* __restrict__ C,
                                                      float* __restrict__ bc, int64_t batch,
                                                      int64_t dstate, int64_t seqlen, int64_t Lp,
                                                      int64_t Bs0, int64_t Bs1, int64_t Bs2,
                                                      int64_t Cs0, int64_t Cs1, int64_t Cs2) {
  const int64_t total = batch * (kGroups * SPL) * Lp;
  for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i < total;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t t = i % Lp;
    const int64_t n = (i / Lp) % (kGroups * SPL);
    const int64_t b = i / (Lp * kGroups * SPL);
    const bool ok = n < dstate && t < seqlen;
    const float bv = ok ? ld<DT>(B, b * Bs0 + n * Bs1 + t * Bs2) : 0.0f;
    const float cv = ok ? ld<DT>(C, b * Cs0 + n * Cs1 + t * Cs2) : 0.0f;
    const int64_t g = n / SPL, k = n % SPL;
    float* o = bc + ((b * kGroups + g) * Lp + t) * (2 * SPL);
    o[k] = bv;
    o[SPL + k] = cv;
  }
}

// ---------------------------------------------------------------------------
template <int DT, int LAYOUT, int SPL>
__global__ __launch_bounds__(kThreads) void scan_kernel(const Params p, const void* __restrict__ u_,
                                                        const void* __restrict__ delta_,
                                                        const void* __restrict__ z_,
                                                        void* __restrict__ y_,
                                                        const float* __restrict__ bc_,
                                                        float* __restrict__ state_out_) {
  using T = typename Ty<DT>::T;
  using V8 = typename Ty<DT>::V8;

  __shared__ __attribute__((aligned(16))) float s_dt[kCPW][kTP];        // delta'
  __shared__ __attribute__((aligned(16))) float s_du[kCPW][kTP];        // delta' * u
  __shared__ __attribute__((aligned(16))) float s_y[kGroups][kCPW][kTP];// partial y

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int g = __builtin_amdgcn_readfirstlane(tid >> 6);  // state group (wave-uniform)
  const int64_t b = blockIdx.y;
  const int64_t d0 = static_cast<int64_t>(blockIdx.x) * kCPW;

  // ---- per-lane recurrence constants ----
  float A2[SPL], h[SPL];
  {
    const int64_t d = d0 + lane;
#pragma unroll
    for (int k = 0; k < SPL; ++k) {
      const int64_t n = static_cast<int64_t>(g) * SPL + k;
      A2[k] = (d < p.dim && n < p.dstate) ? p.A[d * p.As0 + n * p.As1] * kLog2e : 0.0f;
      h[k] = 0.0f;
    }
  }

  // ---- this thread's prologue/epilogue vector: 8 (channel, time) elements ----
  // kTimeContig: channel vc, times vt..vt+7.  kChanContig: channels vc..vc+7, time vt.
  const int vc = (LAYOUT == kTimeContig) ? (tid >> 2) : ((tid >> 5) * kVec);
  const int vt = (LAYOUT == kTimeContig) ? ((tid & 3) * kVec) : (tid & 31);
  auto ec = [&](int j) { return (LAYOUT == kTimeContig) ? vc : vc + j; };
  auto et = [&](int j) { return (LAYOUT == kTimeContig) ? vt + j : vt; };

  const bool has_z = z_ != nullptr;
  float Dv[kVec];
#pragma unroll
  for (int j = 0; j < kVec; ++j) {
    const int64_t d = d0 + ec(j);
    Dv[j] = (p.D != nullptr && d < p.dim) ? p.D[d * p.Ds] : 0.0f;
  }

  V8 ru, rd, rz;
  auto load_raw = [&](int64_t t0) {
    if (p.vec_ok) {
      // The 8 elements are contiguous: one 16-byte (fp16/bf16) or 32-byte (fp32) load.
      const bool in = (d0 + vc < p.dim) && (t0 + vt < p.seqlen);
      const int64_t cu = b * p.us0 + (d0 + vc) * p.us1 + (t0 + vt) * p.us2;
      const int64_t cd = b * p.ds0 + (d0 + vc) * p.ds1 + (t0 + vt) * p.ds2;
      const int64_t cz = b * p.zs0 + (d0 + vc) * p.zs1 + (t0 + vt) * p.zs2;
      V8 zero = {};
      ru = in ? *reinterpret_cast<const V8*>(static_cast<const T*>(u_) + cu) : zero;
      rd = in ? *reinterpret_cast<const V8*>(static_cast<const T*>(delta_) + cd) : zero;
      rz = (in && has_z) ? *reinterpret_cast<const V8*>(static_cast<const T*>(z_) + cz) : zero;
    } else {
#pragma unroll
      for (int j = 0; j < kVec; ++j) {
        const int64_t d = d0 + ec(j), t = t0 + et(j);
        const bool in = d < p.dim && t < p.seqlen;
        ru[j] = in ? static_cast<const T*>(u_)[b * p.us0 + d * p.us1 + t * p.us2] : T(0);
        rd[j] = in ? static_cast<const T*>(delta_)[b * p.ds0 + d * p.ds1 + t * p.ds2] : T(0);
        rz[j] = (in && has_z) ? static_cast<const T*>(z_)[b * p.zs0 + d * p.zs1 + t * p.zs2] : T(0);
      }
    }
  };

  const float* bcw = bc_ + (b * kGroups + g) * p.Lp * (2 * SPL);  // wave-uniform

  if (p.ntiles > 0) load_raw(0);

  for (int64_t tile = 0; tile < p.ntiles; ++tile) {
    const int64_t t0 = tile * kT;

    // ---- prologue: delta', delta'*u -> LDS; D*u and SiLU(z) stay in registers ----
    float yskip[kVec], gate[kVec], dtv[kVec], duv[kVec];
#pragma unroll
    for (int j = 0; j < kVec; ++j) {
      const bool in = (d0 + ec(j) < p.dim) && (t0 + et(j) < p.seqlen);
      const float uu = Ty<DT>::f(ru[j]);
      const float dr = Ty<DT>::f(rd[j]);
      const float dt = p.softplus ? softplus_cut(dr) : dr;
      dtv[j] = in ? dt : 0.0f;  // identity step (a = 1, b = 0) outside the tensor
      duv[j] = in ? dt * uu : 0.0f;
      yskip[j] = Dv[j] * uu;
      gate[j] = has_z ? silu_f(Ty<DT>::f(rz[j])) : 1.0f;
    }
    if (LAYOUT == kTimeContig) {
      float4* pdt = reinterpret_cast<float4*>(&s_dt[vc][vt]);
      float4* pdu = reinterpret_cast<float4*>(&s_du[vc][vt]);
      pdt[0] = make_float4(dtv[0], dtv[1], dtv[2], dtv[3]);
      pdt[1] = make_float4(dtv[4], dtv[5], dtv[6], dtv[7]);
      pdu[0] = make_float4(duv[0], duv[1], duv[2], duv[3]);
      pdu[1] = make_float4(duv[4], duv[5], duv[6], duv[7]);
    } else {
#pragma unroll
      for (int j = 0; j < kVec; ++j) {
        s_dt[vc + j][vt] = dtv[j];
        s_du[vc + j][vt] = duv[j];
      }
    }
    if (tile + 1 < p.ntiles) load_raw(t0 + kT);  // in flight during the scan
    __syncthreads();

    // ---- scan: lane = channel, wave = state group; B/C are SGPR operands ----
    const float* q = bcw + t0 * (2 * SPL);
#pragma unroll 2
    for (int tt = 0; tt < kT; tt += 4) {
      const float4 d4 = *reinterpret_cast<const float4*>(&s_dt[lane][tt]);
      const float4 u4 = *reinterpret_cast<const float4*>(&s_du[lane][tt]);
      const float dts[4] = {d4.x, d4.y, d4.z, d4.w};
      const float dus[4] = {u4.x, u4.y, u4.z, u4.w};
      float ys[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float* qq = q + (tt + j) * (2 * SPL);
        float acc = 0.0f;
#pragma unroll
        for (int k = 0; k < SPL; ++k) {
          const float a = exp2_hw(dts[j] * A2[k]);
          h[k] = __builtin_fmaf(a, h[k], dus[j] * qq[k]);
          acc = __builtin_fmaf(h[k], qq[SPL + k], acc);
        }
        ys[j] = acc;
      }
      *reinterpret_cast<float4*>(&s_y[g][lane][tt]) = make_float4(ys[0], ys[1], ys[2], ys[3]);
    }
    __syncthreads();

    // ---- epilogue: y = (sum_g partial + D*u) * SiLU(z) -> HBM ----
    float yv[kVec];
    if (LAYOUT == kTimeContig) {
#pragma unroll
      for (int j = 0; j < kVec; ++j) yv[j] = yskip[j];
#pragma unroll
      for (int gg = 0; gg < kGroups; ++gg) {
        const float4* py = reinterpret_cast<const float4*>(&s_y[gg][vc][vt]);
        const float4 a0 = py[0], a1 = py[1];
        yv[0] += a0.x; yv[1] += a0.y; yv[2] += a0.z; yv[3] += a0.w;
        yv[4] += a1.x; yv[5] += a1.y; yv[6] += a1.z; yv[7] += a1.w;
      }
    } else {
#pragma unroll
      for (int j = 0; j < kVec; ++j) {
        float s = yskip[j];
#pragma unroll
        for (int gg = 0; gg < kGroups; ++gg) s += s_y[gg][vc + j][vt];
        yv[j] = s;
      }
    }
    V8 ry;
#pragma unroll
    for (int j = 0; j < kVec; ++j) ry[j] = Ty<DT>::from(yv[j] * gate[j]);
    if (p.vec_ok) {
      if ((d0 + vc < p.dim) && (t0 + vt < p.seqlen))
        *reinterpret_cast<V8*>(static_cast<T*>(y_) + b * p.ys0 + (d0 + vc) * p.ys1 +
                               (t0 + vt) * p.ys2) = ry;
    } else {
#pragma unroll
      for (int j = 0; j < kVec; ++j) {
        const int64_t d = d0 + ec(j), t = t0 + et(j);
        if (d < p.dim && t < p.seqlen) static_cast<T*>(y_)[b * p.ys0 + d * p.ys1 + t * p.ys2] = ry[j];
      }
    }
  }

  // ---- final state h[seqlen-1] (selective_scan_chunked.metal:151-155) ----
  if (state_out_ != nullptr) {
    const int64_t d = d0 + lane;
    if (d < p.dim) {
#pragma unroll
      for (int k = 0; k < SPL; ++k) {
        const int64_t n = static_cast<int64_t>(g) * SPL + k;
        if (n < p.dstate) state_out_[(b * p.dim + d) * p.dstate + n] = h[k];
      }
    }
  }
}

// ---------------------------------------------------------------------------
template <int DT, int LAYOUT, int SPL>
void launch(const Params& p, int64_t batch, hipStream_t s) {
  dim3 grid(static_cast<unsigned>(ceil_div(p.dim, kCPW)), static_cast<unsigned>(batch));
  hipLaunchKernelGGL((scan_kernel<DT, LAYOUT, SPL>), grid, dim3(kThreads), 0, s, p, p.u, p.delta,
                     p.z, p.y, p.bc, p.state_out);
}

template <int DT, int LAYOUT>
void launch_spl(const Params& p, int64_t batch, int spl, hipStream_t s) {
  switch (spl) {
    case 1: launch<DT, LAYOUT, 1>(p, batch, s); break;
    case 2: launch<DT, LAYOUT, 2>(p, batch, s); break;
    case 4: launch<DT, LAYOUT, 4>(p, batch, s); break;
    case 8: launch<DT, LAYOUT, 8>(p, batch, s); break;
    default: launch<DT, LAYOUT, 16>(p, batch, s); break;
  }
}

template <int DT>
void launch_layout(const Params& p, int64_t batch, int layout, int spl, hipStream_t s) {
  if (layout == kTimeContig)
    launch_spl<DT, kTimeContig>(p, batch, spl, s);
  else
    launch_spl<DT, kChanContig>(p, batch, spl, s);
}

template <int DT>
void launch_pack(const mm_scan_params* a, int64_t Lp, int spl, hipStream_t s) {
  const int64_t total = a->batch * kGroups * spl * Lp;
  const int64_t blocks = std::min<int64_t>(ceil_div(total, 256), 65536);
  float* bc = static_cast<float*>(a->workspace);
#define MM_PACK(S)                                                                         \
  hipLaunchKernelGGL((pack_bc_kernel<DT, S>), dim3(static_cast<unsigned>(blocks)), dim3(256), \
                     0, s, a->B, a->C, bc, a->batch, a->dstate, a->seqlen, Lp, a->B_stride[0], \
                     a->B_stride[1], a->B_stride[2], a->C_stride[0], a->C_stride[1],        \
                     a->C_stride[2])
  switch (spl) {
    case 1: MM_PACK(1); break;
    case 2: MM_PACK(2); break;
    case 4: MM_PACK(4); break;
    case 8: MM_PACK(8); break;
    default: MM_PACK(16); break;
  }
#undef MM_PACK
}

// Host-side layout analysis: which fast path the four (batch, dim, time) tensors allow.
struct Tens {
  const void* p;
  const int64_t* s;
};

int choose_layout(const mm_scan_params* a, int* layout, int* vec_ok) {
  Tens ts[4] = {{a->u, a->u_stride}, {a->delta, a->delta_stride}, {a->y, a->y_stride},
                {a->z, a->z_stride}};
  const int nt = a->z ? 4 : 3;
  bool time_c = true, chan_c = true;
  for (int i = 0; i < nt; ++i) {
    time_c = time_c && ts[i].s[2] == 1;
    chan_c = chan_c && ts[i].s[1] == 1;
  }
  // Prefer the reference's own layout (time contiguous) when both hold (dim == 1 etc.).
  *layout = time_c ? kTimeContig : chan_c ? kChanContig : kTimeContig;
  bool ok = time_c || chan_c;
  const int64_t es = dtype_size(a->x_dtype);
  const int64_t vbytes = kVec * es;
  if (ok) {
    if (*layout == kTimeContig)
      ok = a->seqlen % kVec == 0;
    else
      ok = a->dim % kVec == 0;
  }
  for (int i = 0; ok && i < nt; ++i) {
    ok = aligned(ts[i].p, vbytes);
    const int64_t other = (*layout == kTimeContig) ? ts[i].s[1] : ts[i].s[2];
    ok = ok && (other % kVec == 0) && (ts[i].s[0] % kVec == 0);
  }
  *vec_ok = ok ? 1 : 0;
  return MM_OK;
}

int validate(const mm_scan_params* a) {
  if (a == nullptr) return fail(MM_ERR_NULL_POINTER, "params is NULL");
  if (!a->u || !a->delta || !a->A || !a->B || !a->C || !a->y)
    return fail(MM_ERR_NULL_POINTER, "u, delta, A, B, C and y are required");
  if (a->batch < 0 || a->dim < 0 || a->seqlen < 0)
    return fail(MM_ERR_SHAPE, "negative size (batch=%lld dim=%lld seqlen=%lld)",
                (long long)a->batch, (long long)a->dim, (long long)a->seqlen);
  if (a->dstate < 1 || a->dstate > MM_MAX_DSTATE)
    return fail(MM_ERR_DSTATE, "dstate=%lld outside [1, %d]", (long long)a->dstate, MM_MAX_DSTATE);
  if (!valid_dtype(a->x_dtype) || !valid_dtype(a->bc_dtype))
    return fail(MM_ERR_DTYPE, "bad dtype (x_dtype=%d bc_dtype=%d)", a->x_dtype, a->bc_dtype);
  if (a->reserved != 0) return fail(MM_ERR_LAYOUT, "reserved field must be 0");
  if (a->batch > 65535) return fail(MM_ERR_SHAPE, "batch=%lld exceeds 65535", (long long)a->batch);
  const size_t need = mm_selective_scan_workspace_size(a->batch, a->dstate, a->seqlen);
  if (need > 0 && (a->workspace == nullptr || a->workspace_bytes < need))
    return fail(MM_ERR_WORKSPACE, "workspace of %zu bytes required, got %zu (%s)", need,
                a->workspace_bytes, a->workspace ? "too small" : "NULL");
  if (a->workspace && !aligned(a->workspace, 16))
    return fail(MM_ERR_WORKSPACE, "workspace must be 16-byte aligned");
  return MM_OK;
}

}  // namespace scan
}  // namespace mm

extern "C" {

size_t mm_selective_scan_workspace_size(int64_t batch, int64_t dstate, int64_t seqlen) {
  using namespace mm::scan;
  if (batch <= 0 || seqlen <= 0 || dstate < 1 || dstate > MM_MAX_DSTATE) return 0;
  const int64_t spl = spl_for(dstate);
  return static_cast<size_t>(batch * kGroups * mm::round_up(seqlen, kT) * 2 * spl) * sizeof(float);
}

int mm_selective_scan_fwd_strided(const mm_scan_params* a, void* stream) {
  using namespace mm;
  using namespace mm::scan;
  clear_error();
  int st = validate(a);
  if (st != MM_OK) return st;
  if (a->batch == 0 || a->dim == 0) return MM_OK;

  int layout = kTimeContig, vec_ok = 0;
  choose_layout(a, &layout, &vec_ok);
  const int spl = spl_for(a->dstate);

  Params p;
  p.u = a->u;
  p.delta = a->delta;
  p.z = a->z;
  p.y = a->y;
  p.A = a->A;
  p.D = a->D;
  p.state_out = a->state_out;
  p.bc = static_cast<const float*>(a->workspace);
  p.dim = a->dim;
  p.dstate = a->dstate;
  p.seqlen = a->seqlen;
  p.Lp = round_up(a->seqlen, kT);
  p.ntiles = p.Lp / kT;
  p.us0 = a->u_stride[0]; p.us1 = a->u_stride[1]; p.us2 = a->u_stride[2];
  p.ds0 = a->delta_stride[0]; p.ds1 = a->delta_stride[1]; p.ds2 = a->delta_stride[2];
  if (a->z) {
    p.zs0 = a->z_stride[0]; p.zs1 = a->z_stride[1]; p.zs2 = a->z_stride[2];
  } else {
    p.zs0 = p.zs1 = p.zs2 = 0;
  }
  p.ys0 = a->y_stride[0]; p.ys1 = a->y_stride[1]; p.ys2 = a->y_stride[2];
  p.As0 = a->A_stride[0];
  p.As1 = a->A_stride[1];
  p.Ds = a->D_stride;
  p.softplus = a->delta_softplus ? 1 : 0;
  p.vec_ok = vec_ok;

  hipStream_t s = static_cast<hipStream_t>(stream);
  if (a->seqlen > 0) {
    switch (a->bc_dtype) {
      case MM_F32: launch_pack<MM_F32>(a, p.Lp, spl, s); break;
      case MM_F16: launch_pack<MM_F16>(a, p.Lp, spl, s); break;
      default: launch_pack<MM_BF16>(a, p.Lp, spl, s); break;
    }
    st = check_launch("pack_bc");
    if (st != MM_OK) return st;
  }
  switch (a->x_dtype) {
    case MM_F32: launch_layout<MM_F32>(p, a->batch, layout, spl, s); break;
    case MM_F16: launch_layout<MM_F16>(p, a->batch, layout, spl, s); break;
    default: launch_layout<MM_BF16>(p, a->batch, layout, spl, s); break;
  }
  return check_launch("selective_scan");
}

int mm_selective_scan_fwd(const void* u, const void* delta, const float* A, const void* B,
                          const void* C, const float* D, const void* z, void* y,
                          float* ssm_state_out, int64_t batch, int64_t dim, int64_t dstate,
                          int64_t seqlen, int32_t x_dtype, int32_t bc_dtype,
                          int32_t delta_softplus, void* workspace, size_t workspace_bytes,
                          void* stream) {
  mm_scan_params a = {};
  a.u = u;
  a.delta = delta;
  a.A = A;
  a.B = B;
  a.C = C;
  a.D = D;
  a.z = z;
  a.y = y;
  a.state_out = ssm_state_out;
  a.workspace = workspace;
  a.workspace_bytes = workspace_bytes;
  a.batch = batch;
  a.dim = dim;
  a.dstate = dstate;
  a.seqlen = seqlen;
  const int64_t xs[3] = {dim * seqlen, seqlen, 1};
  const int64_t bs[3] = {dstate * seqlen, seqlen, 1};
  for (int i = 0; i < 3; ++i) {
    a.u_stride[i] = a.delta_stride[i] = a.z_stride[i] = a.y_stride[i] = xs[i];
    a.B_stride[i] = a.C_stride[i] = bs[i];
  }
  a.A_stride[0] = dstate;
  a.A_stride[1] = 1;
  a.D_stride = 1;
  a.x_dtype = x_dtype;
  a.bc_dtype = bc_dtype;
  a.delta_softplus = delta_softplus;
  return mm_selective_scan_fwd_strided(&a, stream);
}

}  // extern "C"
