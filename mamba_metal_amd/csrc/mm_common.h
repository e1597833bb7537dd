// Shared helpers of libmamba_mi355x: element-type traits, 8-wide vector I/O and
// the thread-local error plumbing behind mm_last_error().
#pragma once

#include <hip/hip_runtime.h>

#include <atomic>
#include <cstdarg>
#include <cstddef>
#include <cstdint>

#include "../../include/mamba_mi355x.h"

namespace mm {

// ---------------------------------------------------------------------------
// Host-side error handling.  Every entry point validates on the host first and
// returns fail(status, ...) before touching HIP; fail() records the message in
// a thread-local buffer read back by mm_last_error().
int fail(int status, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
void clear_error();
// Turns the launch status into MM_OK / MM_ERR_HIP.
int check_launch(const char* what);

inline bool valid_dtype(int32_t dt) { return dt == MM_F32 || dt == MM_F16 || dt == MM_BF16; }
inline int64_t dtype_size(int32_t dt) { return dt == MM_F32 ? 4 : 2; }
inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }
inline int64_t round_up(int64_t a, int64_t b) { return ceil_div(a, b) * b; }
inline bool aligned(const void* p, int64_t bytes) {
  return (reinterpret_cast<uintptr_t>(p) % static_cast<uintptr_t>(bytes)) == 0;
}

// Per-device cache of a launch constant (CU count, resident workgroups per CU of one
// kernel).  The value is computed on first use on each device and published with an
// atomic store; racing threads compute and store the same value, so no lock is needed.
constexpr int kMaxDevices = 64;
struct DeviceCache {
  std::atomic<int> v[kMaxDevices];
};
template <typename F>
int device_cached(DeviceCache& c, F compute, int fallback) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    const int x = compute();  // uncached, same fallback
    return x < 1 ? fallback : x;
  }
  int x = c.v[dev].load(std::memory_order_relaxed);
  if (x == 0) {
    x = compute();
    if (x < 1) x = fallback;
    c.v[dev].store(x, std::memory_order_relaxed);
  }
  return x;
}
// Compute units of the current device.
int num_cus();

// ---------------------------------------------------------------------------
// Device-side element types.  All arithmetic is fp32; T is the storage type.
typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef unsigned short ushort8_t __attribute__((ext_vector_type(8)));
typedef float float8_t __attribute__((ext_vector_type(8)));

__device__ __forceinline__ float bf16_to_f32(unsigned short v) {
  return __uint_as_float(static_cast<uint32_t>(v) << 16);
}
// Round-to-nearest-even fp32 -> bf16; NaN stays NaN (quiet bit set).
__device__ __forceinline__ unsigned short f32_to_bf16(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return static_cast<unsigned short>((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return static_cast<unsigned short>(u >> 16);
}

template <int DT>
struct Ty;

template <>
struct Ty<MM_F32> {
  using T = float;
  using V8 = float8_t;
  __device__ static __forceinline__ float f(T x) { return x; }
  __device__ static __forceinline__ T from(float x) { return x; }
};

template <>
struct Ty<MM_F16> {
  using T = _Float16;
  using V8 = half8_t;
  __device__ static __forceinline__ float f(T x) { return static_cast<float>(x); }
  __device__ static __forceinline__ T from(float x) { return static_cast<_Float16>(x); }
};

template <>
struct Ty<MM_BF16> {
  using T = unsigned short;
  using V8 = ushort8_t;
  __device__ static __forceinline__ float f(T x) { return bf16_to_f32(x); }
  __device__ static __forceinline__ T from(float x) { return f32_to_bf16(x); }
};

template <int DT>
__device__ __forceinline__ float ld(const void* p, int64_t i) {
  return Ty<DT>::f(static_cast<const typename Ty<DT>::T*>(p)[i]);
}
template <int DT>
__device__ __forceinline__ void st(void* p, int64_t i, float v) {
  static_cast<typename Ty<DT>::T*>(p)[i] = Ty<DT>::from(v);
}

// Fast-math building blocks on the hardware transcendental unit.
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

__device__ __forceinline__ float exp2_hw(float x) { return __builtin_amdgcn_exp2f(x); }
__device__ __forceinline__ float log2_hw(float x) { return __builtin_amdgcn_logf(x); }

// 2^x to ~1 ulp without a one-sided bias: 2^n * 2^r with n = rint(x) and r = x - n in
// [-1/2, 1/2] (exact), 2^r from its Taylor series sum_k (r ln 2)^k / k! to k = 7 (the
// dropped terms are < 1e-8 relative), Horner with fma.  A decay exp2(delta2 * A) enters
// the state once per step, so over a state's memory (thousands of steps when |A| delta is
// ~1e-3) a per-step error that always leans one way adds up linearly; v_exp_f32's does
// and moves long fp32 scans by ~1e-5 relative, this one's rounding errors do not.
__device__ __forceinline__ float exp2_acc(float x) {
  x = fminf(fmaxf(x, -160.0f), 128.0f);  // past either end the result is 0 or +inf anyway
  const float n = __builtin_rintf(x);
  const float r = x - n;
  float q = 1.5252733804059840e-05f;      // (ln 2)^7 / 7!
  q = __builtin_fmaf(q, r, 1.5403530393381606e-04f);  // (ln 2)^6 / 6!
  q = __builtin_fmaf(q, r, 1.3333558146428443e-03f);  // (ln 2)^5 / 5!
  q = __builtin_fmaf(q, r, 9.6181291076284772e-03f);  // (ln 2)^4 / 4!
  q = __builtin_fmaf(q, r, 5.5504108664821580e-02f);  // (ln 2)^3 / 3!
  q = __builtin_fmaf(q, r, 2.4022650695910071e-01f);  // (ln 2)^2 / 2!
  q = __builtin_fmaf(q, r, 6.9314718055994531e-01f);  // ln 2
  q = __builtin_fmaf(q, r, 1.0f);
  return __builtin_ldexpf(q, static_cast<int>(n));
}

// The scan's decay: fp32 inputs take exp2_acc (parity at rtol 1e-5 over long
// sequences); fp16 / bf16 inputs (tolerance 1e-3) take v_exp_f32.
template <int DT>
__device__ __forceinline__ float exp2_decay(float x) {
  if constexpr (DT == MM_F32) return exp2_acc(x);
  else return exp2_hw(x);
}
__device__ __forceinline__ float rcp_hw(float x) { return __builtin_amdgcn_rcpf(x); }

// RMSNorm output element: round(x * inv * w) to DT with the fp32 product rounded first.
// The empty asm makes the fp32 product an opaque register value, so instruction selection
// cannot fuse the last multiply and the conversion into one single-rounding
// mixed-precision instruction (v_fma_mixlo_f16, which it otherwise picks in some kernels
// and not others): every RMSNorm site -- the norm kernels and the GEMMs that normalise
// their operand on load -- then rounds identically.
template <int DT>
__device__ __forceinline__ typename Ty<DT>::T norm_round(float x, float inv, float w) {
  float t = x * inv * w;
  asm("" : "+v"(t));
  return Ty<DT>::from(t);
}

// silu(z) = z * sigmoid(z) (selective_scan_chunked.metal:143).
__device__ __forceinline__ float silu_f(float z) { return z * rcp_hw(1.0f + exp2_hw(-z * kLog2e)); }

// v of lane (lane ^ m) within the wave, for m = 1, 2, 4, 8, 16, 32, on VALU cross-lane
// operations instead of an LDS permute (ds_bpermute, a ~100-cycle round trip on the
// reductions' critical path): DPP quad permutes for 1 and 2, the half-row mirror
// (lane ^ 7) then a quad reverse (^ 3) for 4, a 16-lane row rotation by 8 for 8, and
// gfx950's v_permlane16 / v_permlane32 swaps (which hand both halves to every lane) for
// 16 and 32.  The whole wave must be active, as at every call site.
template <int CTRL>
__device__ __forceinline__ float dpp_mov(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ float lane_xor(float v, int m) {
  switch (m) {
    case 1: return dpp_mov<0xB1>(v);                    // quad_perm [1,0,3,2]
    case 2: return dpp_mov<0x4E>(v);                    // quad_perm [2,3,0,1]
    case 4: return dpp_mov<0x1B>(dpp_mov<0x141>(v));    // half-row mirror, quad_perm [3,2,1,0]
    case 8: return dpp_mov<0x128>(v);                   // row_ror:8
    case 16: {
      const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
      return __uint_as_float((__lane_id() & 16) ? r[0] : r[1]);
    }
    case 32: {
      const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
      return __uint_as_float((__lane_id() & 32) ? r[0] : r[1]);
    }
    default: return __shfl_xor(v, m, 64);
  }
}

// log(1 + exp(x)), the softplus below the reference's cutoff of 20
// (selective_scan_chunked.metal:60-65; the scan applies the cutoff itself).  log1p is
// evaluated as log(s) * e / (s - 1) with s = 1 + e (Goldberg's log1p correction) so tiny
// e keeps full relative precision.
__device__ __forceinline__ float log1p_exp(float x) {
  const float e = exp2_hw(x * kLog2e);
  const float s = 1.0f + e;
  const float dm = s - 1.0f;
  const float l = log2_hw(s) * kLn2;
  return (dm == 0.0f) ? e : l * (e * rcp_hw(dm));
}

// softplus without cutoff: log(1 + exp(x)) = max(x, 0) + log1p(exp(-|x|))
// (MLX nn.softplus used by MambaBlock.step, mamba_block.py:184).
__device__ __forceinline__ float softplus_full(float x) {
  const float e = exp2_hw(-fabsf(x) * kLog2e);
  const float s = 1.0f + e;
  const float dm = s - 1.0f;
  const float l = log2_hw(s) * kLn2;
  const float lp = (dm == 0.0f) ? e : l * (e * rcp_hw(dm));
  return fmaxf(x, 0.0f) + lp;
}

}  // namespace mm
