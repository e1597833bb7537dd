// Weight-streaming GEMM for the decode step: mm_decode_linear, mm_pack_linear_weight.
//
//   Y[M, N] = X[M, K] . W[N, K]^T          (M <= 64 rows: one token per sequence)
//
// covers the nn.Linear projections of MambaBlock.step (in_proj, x_proj, out_proj;
// mamba_metal/mamba_block.py:166-196) and the tied LM head (mamba_model.py:78) at
// decode batch M.  With M <= 64 each weight element is used M times and read once:
// the kernel is HBM-bound on N*K*elem bytes of W.
//
// Packed weights.  W is repacked once (mm_pack_linear_weight) into the operand
// order of v_mfma_f32_32x32x16: block (t, s) of 1 KB holds, for lane l, the 8
// elements W[32t + l%32, 16s + 8(l/32) .. +7].  A wave's W load for one MFMA step
// is then one 1 KB contiguous read -- the access pattern of a plain stream.
//
// X goes through LDS: 64-row x 64-k chunks of X are loaded with 128-byte row
// segments (8 rows per load instruction), written to an LDS tile (rows padded to 144
// bytes) and the MFMA A operands are read from there.
//
// Work split.  X is as large as 64 columns of W (M = 64), and every workgroup that
// covers a K range re-reads that range of X from L2; measured on MI355X that traffic
// costs about as much as the weight stream itself, so the split is chosen to share it:
//   * very wide N (> 512 column tiles): share_kernel -- NW waves own NW adjacent
//     32-column tiles, walk all of K together and share one X chunk per step through LDS;
//   * otherwise linear_kernel, NT 32-column tiles per workgroup (NT = 2 from 256 tiles
//     on): with enough tiles (or a small weight share) K stays in the workgroup, its KSW
//     waves split K and their partial tiles meet in LDS (summed in fixed wave order)
//     before the epilogue.
//     Narrow calls split K over the grid's y dimension instead: workgroups write fp32
//     partial tiles, row-major [split][M][N], to the workspace, and a second kernel
//     sums the splits in order and runs the epilogue -- deterministic, and the kernel
//     boundary orders the partials without any cross-workgroup protocol.  With >= 16
//     column tiles the split workgroups are share_kernel's (4 waves sharing X, up to 8
//     splits); below that, single-wave linear_kernel workgroups;
//   * M <= 4: gemv_kernel (below), 8 output columns per workgroup over all CUs.
//
// Input RMSNorm (x_norm_w set, M <= 8, linear_kernel only): X holds the raw residual
// rows; every wave first computes each row's inverse RMS exactly as
// add_rmsnorm_vec_kernel does (same chunk order, fma chain and shuffle tree), then
// scales the X operand rows by it and by the norm weight before the LDS write, so the
// product sees the same rounded operand as after a separate norm pass.  At small batch
// this drops the norm kernel between out_proj and the next in_proj.
//
// Epilogues fold the decode step's neighbouring element-wise ops into the GEMM:
//   MM_LIN_STORE  y[m, n] = acc
//   MM_LIN_RESID  resid[m, n] = resid[m, n] + round(acc)     (out_proj + residual,
//                 mamba_model.py:48 -- the residual stream stays in x's dtype)
//   MM_LIN_CONV   in_proj + conv window: for n < n_conv the rounded acc is the new
//                 conv input x[m, n]: the (M, n_conv, 4) conv state shifts in place
//                 and conv_out[m, n] = silu(bias + w . window) (mamba_block.py:
//                 172-179); for n >= n_conv, y[m, n - n_conv] = acc (the z half).
#include "mm_common.h"

namespace mm {
namespace gemm {

constexpr int kTileN = 32;
constexpr int kStepK = 16;
constexpr int kChunkK = 64;               // K per LDS chunk = 4 MFMA steps
constexpr int kSteps = kChunkK / kStepK;
constexpr int kMaxM = 64;
constexpr int kRowBytes = kChunkK * 2 + 16;  // padded LDS row of one X chunk
constexpr int kXLds = kMaxM * kRowBytes;     // 9216 B per wave for the X chunk
constexpr int kPartial = 4;                  // internal "epilogue": write fp32 partials
constexpr int kStoreArgmax = 6;              // share_kernel: STORE + per-row argmax candidates
constexpr int kShareTiles = 512;             // wider N runs the shared-X kernel
constexpr int kNormInMaxM = 8;               // input RMSNorm: rows of X load instruction 0
constexpr int kNormInMaxK = 4096;            // input RMSNorm: rows add_rmsnorm_vec_kernel takes

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

template <int DT>
__device__ __forceinline__ f32x16 mfma(u32x4 a, u32x4 b, f32x16 c) {
  if constexpr (DT == MM_F16)
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}

struct LinParams {
  const void* x;
  const void* w;  // packed
  void* y;
  void* resid;
  void* conv_state;
  const void* conv_w;
  const void* conv_b;
  void* conv_out;
  const void* norm_w;
  void* norm_out;
  float* partials;  // split calls: [ks][M][N] fp32
  const void* x_norm_w;  // input RMSNorm weight (K,), or null
  // x_proj folded into in_proj's conv epilogue (mm_decode_in_proj_xproj): packed
  // x_proj weight (xp_n rows, K = n_conv, xp_nsteps 16-k steps), fp32 partial planes
  // [n_conv / TN][M][xp_n] and the (M, xp_n) output.
  const u32x4* xp_w;
  float* xp_part;
  void* xp_y;
  int64_t xp_n, xp_nsteps, ld_xp;
  int64_t M, N, K, ldx, ldy, ldr, ldc, ldn, n_conv;
  float eps, x_eps;
  int32_t ks;       // K splits across workgroups (grid.y)
  // kStoreArgmax: per (workgroup, row) the best stored logit and its column,
  // cand_v[blockIdx.x * M + m] / cand_i[...]
  float* cand_v;
  int32_t* cand_i;
};

struct Plan {
  int nt, ks, ksw;
  int nw;  // > 0: shared-X kernel with nw waves splitting N (nt = ks = ksw = 1)
};

// Launch shape (from sweeps on MI355X over the decode shapes of Mamba-130M..2.8B).
// Very wide N (> 512 32-column tiles: the LM head) runs the shared-X kernel: NW waves
// split the workgroup's NW x 32 columns, walk all of K together and stage each X chunk
// in LDS once for all of them, a quarter (NW = 4) or an eighth (NW = 8) of the X
// traffic per weight byte; NW keeps the grid within 256 workgroups.  For 256..512
// tiles (in_proj of the large models) a wave owns NT = 2 tiles, so each X operand
// feeds two MFMAs.  K stays in the workgroup (up to 4 waves splitting it) when there
// are >= 128 workgroups' worth of column tiles or when one workgroup's share of W is
// small (<= 160 KB: a second kernel for a split-K reduction costs more than it saves,
// which is the batch-1 decode case); otherwise K is split over single-wave workgroups
// until ~640 of them fill the chip, each keeping >= 2 chunks of K.
inline Plan plan(int64_t N, int64_t K) {
  const int64_t nchunks = K / kChunkK;
  Plan p{1, 1, 1, 0};
  const int64_t nt32 = ceil_div(N, kTileN);
  if (nt32 > kShareTiles) {
    p.nw = nt32 <= 1024 ? 4 : 8;
    return p;
  }
  if (nt32 >= 256) p.nt = 2;
  const int64_t ntiles = ceil_div(N, kTileN * p.nt);
  const int64_t wg_bytes = kTileN * p.nt * K * 2;
  if (ntiles >= 128 || wg_bytes <= (160 << 10)) {
    while (p.ksw < 4 && ntiles * p.ksw < 512 && nchunks / (p.ksw * 2) >= 2) p.ksw *= 2;
  } else if (nt32 >= 16) {
    // K split with X shared by 4 waves over 128 columns: single-wave split workgroups
    // re-read their K range of X once per 32-column tile, which at M = 64 is twice the
    // weight bytes (2.8B out_proj: 52 MB of X for 26 MB of W); sharing cuts it 4x.
    // Splits double up to 8 while the grid is under 256 workgroups and each keeps >= 2
    // chunks.  Measured at the 2.8B out_proj shape (+ residual + norm pass): 8 splits
    // (160 workgroups of 10 chunks) 14.5 us; 16 splits 18.0; 4 splits 17.7; 8 waves x 8 or
    // 16 splits 17.9 / 16.6; single-wave 8-way split (640 workgroups) 16.2.
    p.nw = 4;
    const int64_t groups = ceil_div(nt32, 4);
    while (p.ks < 8 && groups * p.ks < 256 && nchunks / (p.ks * 2) >= 2) p.ks *= 2;
  } else {
    while (p.ks < 64 && ntiles * p.ks < 640 && nchunks / (p.ks * 2) >= 2) p.ks *= 2;
  }
  return p;
}

template <int DT, int EPI>
__device__ __forceinline__ void epilogue(const LinParams& p, int64_t m, int64_t n, float v) {
  using T = typename Ty<DT>::T;
  if constexpr (EPI == MM_LIN_STORE) {
    st<DT>(p.y, m * p.ldy + n, v);
  } else if constexpr (EPI == MM_LIN_RESID) {
    T* r = static_cast<T*>(p.resid) + m * p.ldr + n;
    *r = Ty<DT>::from(Ty<DT>::f(*r) + Ty<DT>::f(Ty<DT>::from(v)));
  } else {
    if (n < p.n_conv) {
      typedef T T4 __attribute__((ext_vector_type(4)));
      T4* sp = static_cast<T4*>(p.conv_state) + m * p.n_conv + n;
      const T4 win = *sp;
      const T4 cw = static_cast<const T4*>(p.conv_w)[n];
      const T xr = Ty<DT>::from(v);
      float a = p.conv_b ? ld<DT>(p.conv_b, n) : 0.0f;
      a = __builtin_fmaf(Ty<DT>::f(cw[0]), Ty<DT>::f(win[1]), a);
      a = __builtin_fmaf(Ty<DT>::f(cw[1]), Ty<DT>::f(win[2]), a);
      a = __builtin_fmaf(Ty<DT>::f(cw[2]), Ty<DT>::f(win[3]), a);
      a = __builtin_fmaf(Ty<DT>::f(cw[3]), Ty<DT>::f(xr), a);
      T4 nw;
      nw[0] = win[1];
      nw[1] = win[2];
      nw[2] = win[3];
      nw[3] = xr;
      *sp = nw;
      st<DT>(p.conv_out, m * p.ldc + n, silu_f(a));
    } else {
      st<DT>(p.y, m * p.ldy + (n - p.n_conv), v);
    }
  }
}

// One lane's part of a row's sum of squares in add_rmsnorm_vec_kernel's order: lane
// takes 8-element chunks lane + 64 i (i < kNormChunks: rows of up to 4096 elements),
// squares accumulated by fma in (i, k) order, chunks past the row counted as zeros.  All
// chunk loads are issued (clamped to chunk 0) before the first is used.
constexpr int kNormChunks = 8;
static_assert(kNormChunks * 64 * 8 == kNormInMaxK, "row_sumsq covers rows of kNormInMaxK elements");

template <int DT>
__device__ __forceinline__ float row_sumsq(const typename Ty<DT>::T* r, int nch, int lane) {
  using V8 = typename Ty<DT>::V8;
  V8 v[kNormChunks];
#pragma unroll
  for (int i = 0; i < kNormChunks; ++i) {
    const int ch = lane + 64 * i;
    v[i] = *reinterpret_cast<const V8*>(r + 8 * (ch < nch ? ch : 0));
  }
  float ss = 0.0f;
#pragma unroll
  for (int i = 0; i < kNormChunks; ++i) {
    const bool ok = lane + 64 * i < nch;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const float x = ok ? Ty<DT>::f(v[i][k]) : 0.0f;
      ss = __builtin_fmaf(x, x, ss);
    }
  }
  return ss;
}

// MFMA output layout: lane l, register i of a 32x32 tile holds row
// 8*(i/4) + 4*(l/32) + i%4, column l%32.
__device__ __forceinline__ int acc_row(int i, int lane) { return 8 * (i >> 2) + 4 * (lane >> 5) + (i & 3); }

// LDS of one linear_kernel workgroup: a per-wave slot that holds the X chunk during the
// K loop and the wave's partial tiles afterwards.
template <int KSW, int MT, int NT, int EPI>
struct LinLds {
  static constexpr int kNacc = MT * NT * 16;  // accumulator floats per lane
  static constexpr int kWave = kXLds > kNacc * 64 * 4 ? kXLds : kNacc * 64 * 4;
  static constexpr int kBytes = (EPI == kPartial ? 1 : KSW) * kWave;
};

// The body of linear_kernel for column block t (TN = NT * 32 columns from t * TN) and K
// split ks, on the workgroup's LDS block smem (LinLds bytes).  kZStore is the STORE
// epilogue of the z half of in_proj (columns from n_conv on, stored to y[m, n - n_conv]).
constexpr int kZStore = 5;

template <int DT, int KSW, int MT, int NT, int EPI, bool NORM = false, bool XP = false>
__device__ __forceinline__ void linear_body(const LinParams& p, const int64_t t, const int ks,
                                            char* const smem) {
  using T = typename Ty<DT>::T;
  using V8 = typename Ty<DT>::V8;
  static_assert(!NORM || MT == 1, "the input RMSNorm covers rows 0..7 of one m-tile");
  static_assert(!XP || (EPI == MM_LIN_CONV && KSW == 4 && !NORM), "x_proj rides the 4-wave conv epilogue");
  constexpr int XI = MT * 4;                 // X load instructions per chunk (8 rows each)
  constexpr int NACC = MT * NT * 16;         // accumulator floats per lane
  constexpr int kWaveLds = LinLds<KSW, MT, NT, EPI>::kWave;
  constexpr int TN = NT * kTileN;            // columns per workgroup
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  char* const xs = smem + (EPI == kPartial ? 0 : wave * kWaveLds);
  const int64_t n0 = t * TN;
  const int64_t nsteps = p.K / kStepK;
  const int64_t nchunks = p.K / kChunkK;
  // chunk range of this workgroup, then of this wave
  const int64_t per_wg = (nchunks + p.ks - 1) / p.ks;
  const int64_t g0 = ks * per_wg;
  const int64_t g1 = g0 + per_wg < nchunks ? g0 + per_wg : nchunks;
  const int64_t per_w = (g1 - g0 + KSW - 1) / KSW;
  const int64_t c_begin = g0 + wave * per_w;
  const int64_t c_end = c_begin + per_w < g1 ? c_begin + per_w : g1;

  // Every global load is unconditional and in bounds (chunks past this wave's range
  // re-read its last chunk, rows past M read row 0, column tiles past N read tile 0
  // -- all of which only feed outputs that are never stored), so the compiler
  // counts outstanding loads exactly.
  const int64_t ntiles32 = (p.N + kTileN - 1) / kTileN;
  const u32x4* wp[NT];
#pragma unroll
  for (int j = 0; j < NT; ++j) {
    const int64_t tj = t * NT + j;
    wp[j] = static_cast<const u32x4*>(p.w) + (tj < ntiles32 ? tj : 0) * nsteps * 64 + lane;
  }
  const T* xrow[XI];
#pragma unroll
  for (int i = 0; i < XI; ++i) {
    const int64_t r = 8 * i + (lane >> 3);
    xrow[i] = static_cast<const T*>(p.x) + (r < p.M ? r : 0) * p.ldx + 8 * (lane & 7);
  }
  // LDS slots: write (row 8i + l/8, 16-byte column l%8); read for step g, m-tile mt:
  // row 32mt + l%32, column 2g + l/32.
  const int wr_off = (lane >> 3) * kRowBytes + (lane & 7) * 16;

  // Input RMSNorm: inverse RMS of row l/8 (the rows of X load instruction 0; the host
  // guarantees M <= 8), computed per row by the whole wave in add_rmsnorm_vec_kernel's
  // order: lane takes 8-element chunks lane + 64 i, squares accumulate by fma in (i, k)
  // order, then the xor-shuffle tree 32, 16, ..., 1.  Run after the first chunk's
  // loads are issued, so the two latencies overlap.
  float xinv = 0.0f;
  auto input_norm = [&]() __attribute__((always_inline)) {
    const int nch = static_cast<int>(p.K >> 3);
    for (int64_t m = 0; m < p.M; ++m) {
      const T* const r = static_cast<const T*>(p.x) + m * p.ldx;
      float ss = row_sumsq<DT>(r, nch, lane);
#pragma unroll
      for (int off = 32; off > 0; off >>= 1) ss += lane_xor(ss, off);
      const float inv = rsqrtf(ss / static_cast<float>(p.K) + p.x_eps);
      if ((lane >> 3) == m) xinv = inv;
    }
  };
  const int rd_off = (lane & 31) * kRowBytes + (lane >> 5) * 16;

  // Epilogue ownership (reduced tile element e = row * TN + col, e = tid + u * KSW * 64):
  // the column is the same for all of a thread's elements (KSW * 64 is a multiple of TN),
  // the rows step by KSW * 64 / TN.  The conv epilogue's inputs (window, weights, bias)
  // do not depend on the product: they are loaded before the K loop so their latency
  // hides under it (clamped: elements outside the conv half read column 0, row 0).
  constexpr int EPT = EPI == kPartial ? 1 : MT * 32 * TN / (KSW * 64);
  static_assert(EPI == kPartial || (KSW * 64) % TN == 0, "epilogue column per thread");
  const int e_col = threadIdx.x % TN;
  const int e_row0 = threadIdx.x / TN;
  constexpr int kRowStep = KSW * 64 / TN;
  typedef T T4 __attribute__((ext_vector_type(4)));
  T4 win[EPI == MM_LIN_CONV ? EPT : 1];
  T4 cw{};
  float cbias = 0.0f;
  if constexpr (EPI == MM_LIN_CONV) {
    const int64_t n = n0 + e_col;
    const int64_t nc = n < p.n_conv ? n : 0;
    const T4* const sb = static_cast<const T4*>(p.conv_state);
#pragma unroll
    for (int u = 0; u < EPT; ++u) {
      const int64_t m = e_row0 + u * kRowStep;
      win[u] = sb[(m < p.M ? m : 0) * p.n_conv + nc];
    }
    cw = static_cast<const T4*>(p.conv_w)[nc];
    if (p.conv_b) cbias = Ty<DT>::f(static_cast<const T*>(p.conv_b)[nc]);
  }

  f32x16 acc[MT][NT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int j = 0; j < NT; ++j)
#pragma unroll
      for (int i = 0; i < 16; ++i) acc[mt][j][i] = 0.0f;

  if (c_begin < c_end) {
    const int64_t c_last = c_end - 1;
    u32x4 wa[NT][kSteps], xa[XI], wb[NT][kSteps], xb[XI];
    u32x4 na = {0u, 0u, 0u, 0u}, nb = na;  // input-norm weight chunk (NORM)
    auto load = [&](u32x4(&wv)[NT][kSteps], u32x4(&xv)[XI], u32x4& nv, int64_t c) {
      const int64_t cc = c < c_end ? c : c_last;
#pragma unroll
      for (int j = 0; j < NT; ++j)
#pragma unroll
        for (int g = 0; g < kSteps; ++g) wv[j][g] = wp[j][(cc * kSteps + g) * 64];
#pragma unroll
      for (int i = 0; i < XI; ++i) xv[i] = *reinterpret_cast<const u32x4*>(xrow[i] + cc * kChunkK);
      if constexpr (NORM)
        nv = *reinterpret_cast<const u32x4*>(static_cast<const T*>(p.x_norm_w) + cc * kChunkK +
                                             8 * (lane & 7));
    };
    auto compute = [&](const u32x4(&wv)[NT][kSteps], const u32x4(&xv)[XI], const u32x4& nv,
                       int64_t c) {
      if (c >= c_end) return;
#pragma unroll
      for (int i = 0; i < XI; ++i) {
        u32x4 v = xv[i];
        if constexpr (NORM) {
          if (i == 0) {  // rows 0..7: round(x * inv * w), add_rmsnorm_vec_kernel's expression
            const V8 xr = __builtin_bit_cast(V8, v);
            const V8 wr = __builtin_bit_cast(V8, nv);
            V8 o;
#pragma unroll
            for (int k = 0; k < 8; ++k) o[k] = norm_round<DT>(Ty<DT>::f(xr[k]), xinv, Ty<DT>::f(wr[k]));
            v = __builtin_bit_cast(u32x4, o);
          }
        }
        *reinterpret_cast<u32x4*>(xs + 8 * i * kRowBytes + wr_off) = v;
      }
      // LDS is in order per wave: the reads below see the writes above; this only
      // keeps the compiler from moving them across.
      __builtin_amdgcn_wave_barrier();
#pragma unroll
      for (int g = 0; g < kSteps; ++g)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          const u32x4 a = *reinterpret_cast<const u32x4*>(xs + mt * 32 * kRowBytes + rd_off + g * 32);
#pragma unroll
          for (int j = 0; j < NT; ++j) acc[mt][j] = mfma<DT>(a, wv[j][g], acc[mt][j]);
        }
      __builtin_amdgcn_wave_barrier();
    };

    load(wa, xa, na, c_begin);
    if constexpr (NORM) input_norm();
    // The last one or two chunks are peeled off: the loop body's prefetch of chunk c + 2
    // would re-read the last chunk once more (measured: 2.8B decode 3.665 -> 3.642 ms).
    int64_t c = c_begin;
    for (; c + 2 < c_end; c += 2) {
      load(wb, xb, nb, c + 1);
      compute(wa, xa, na, c);
      load(wa, xa, na, c + 2);
      compute(wb, xb, nb, c + 1);
    }
    load(wb, xb, nb, c + 1);
    compute(wa, xa, na, c);
    compute(wb, xb, nb, c + 1);
  }

  if constexpr (EPI == kPartial) {
    // Single-wave workgroup: write the raw tile to partials[ks] (row-major), a row
    // segment of 32 consecutive floats per half-wave and register.
    float* const dst = p.partials + static_cast<int64_t>(ks) * p.M * p.N;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int j = 0; j < NT; ++j)
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int64_t m = 32 * mt + acc_row(i, lane);
          const int64_t n = n0 + 32 * j + (lane & 31);
          if (m < p.M && n < p.N) dst[m * p.N + n] = acc[mt][j][i];
        }
    return;
  } else {
    // XP: this wave's x_proj weight tiles (32 rows each, waves w and w + 4), loaded
    // here so that their latency overlaps the partial-tile exchange and the conv step.
    constexpr int XPT = 2;                 // x_proj column tiles per wave (xp_n <= 256)
    constexpr int XST = TN / kStepK;       // x_proj k steps of this workgroup (its TN columns)
    u32x4 wx[XP ? XPT : 1][XP ? XST : 1];
    const bool xp_here = XP && n0 < p.n_conv;  // workgroup-uniform (n_conv % TN == 0)
    if constexpr (XP) {
      const int64_t ntx = (p.xp_n + kTileN - 1) / kTileN;
      const int64_t s0 = n0 / kStepK;
#pragma unroll
      for (int i = 0; i < XPT; ++i) {
        const int64_t j = wave + 4 * i;
        const int64_t jj = j < ntx && xp_here ? j : 0;
#pragma unroll
        for (int g = 0; g < XST; ++g) wx[i][g] = p.xp_w[(jj * p.xp_nsteps + (xp_here ? s0 : 0) + g) * 64 + lane];
      }
    }
    // Partial tiles -> this wave's LDS slot (register-major, lane-contiguous).
    float* const part = reinterpret_cast<float*>(xs);
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int j = 0; j < NT; ++j)
#pragma unroll
        for (int i = 0; i < 16; ++i) part[((mt * NT + j) * 16 + i) * 64 + lane] = acc[mt][j][i];
    __syncthreads();
    // Tile element e = row * TN + col, summed over the waves in order.  Each thread
    // takes EPT elements; the residual loads for all of them are issued before any
    // of them is used.
    float vals[EPT];
    int64_t ms[EPT], ns[EPT];
#pragma unroll
    for (int u = 0; u < EPT; ++u) {
      const int row = e_row0 + u * kRowStep, col = e_col;
      const int rr = row & 31;
      const int reg = (((row >> 5) * NT + (col >> 5)) * 16) + 4 * (rr >> 3) + (rr & 3);
      const int ln = (col & 31) + 32 * ((rr >> 2) & 1);
      float v = 0.0f;
#pragma unroll
      for (int w = 0; w < KSW; ++w)
        v += reinterpret_cast<const float*>(smem + w * kWaveLds)[reg * 64 + ln];
      vals[u] = v;
      ms[u] = row;
      ns[u] = n0 + col;
    }
    if constexpr (EPI == MM_LIN_STORE || EPI == kZStore) {
      const int64_t c0 = EPI == kZStore ? p.n_conv : 0;
#pragma unroll
      for (int u = 0; u < EPT; ++u)
        if (ms[u] < p.M && ns[u] < p.N) st<DT>(p.y, ms[u] * p.ldy + ns[u] - c0, vals[u]);
    } else if constexpr (EPI == MM_LIN_RESID) {
      T* const rb = static_cast<T*>(p.resid);
      T old[EPT];
#pragma unroll
      for (int u = 0; u < EPT; ++u) {
        const bool ok = ms[u] < p.M && ns[u] < p.N;
        old[u] = rb[ok ? ms[u] * p.ldr + ns[u] : 0];
      }
#pragma unroll
      for (int u = 0; u < EPT; ++u)
        if (ms[u] < p.M && ns[u] < p.N)
          rb[ms[u] * p.ldr + ns[u]] = Ty<DT>::from(Ty<DT>::f(old[u]) + Ty<DT>::f(Ty<DT>::from(vals[u])));
    } else {
      T4* const sb = static_cast<T4*>(p.conv_state);
      T cov[XP ? EPT : 1];  // XP: this thread's conv outputs, the x_proj operand
#pragma unroll
      for (int u = 0; u < (XP ? EPT : 1); ++u) cov[u] = Ty<DT>::from(0.0f);
#pragma unroll
      for (int u = 0; u < EPT; ++u) {
        const int64_t m = ms[u], n = ns[u];
        if (m >= p.M || n >= p.N) continue;
        if (n < p.n_conv) {
          const T xr = Ty<DT>::from(vals[u]);
          float a = cbias;
          a = __builtin_fmaf(Ty<DT>::f(cw[0]), Ty<DT>::f(win[u][1]), a);
          a = __builtin_fmaf(Ty<DT>::f(cw[1]), Ty<DT>::f(win[u][2]), a);
          a = __builtin_fmaf(Ty<DT>::f(cw[2]), Ty<DT>::f(win[u][3]), a);
          a = __builtin_fmaf(Ty<DT>::f(cw[3]), Ty<DT>::f(xr), a);
          T4 nw;
          nw[0] = win[u][1];
          nw[1] = win[u][2];
          nw[2] = win[u][3];
          nw[3] = xr;
          sb[m * p.n_conv + n] = nw;
          const T co = Ty<DT>::from(silu_f(a));
          static_cast<T*>(p.conv_out)[m * p.ldc + n] = co;
          if constexpr (XP) cov[u] = co;
        } else {
          st<DT>(p.y, m * p.ldy + (n - p.n_conv), vals[u]);
        }
      }
      if constexpr (XP) {
        if (xp_here) {
          // x_proj partial of this workgroup's K range (its TN conv columns):
          // part[t][m][n] = sum_k conv_out[m, n0 + k] * W_x[n, n0 + k].  The conv
          // outputs go to LDS (slot 0, the X-chunk layout) as the MFMA A operand.
          __syncthreads();  // every wave has read the partial-sum slots
          T* const xt = reinterpret_cast<T*>(smem);
#pragma unroll
          for (int u = 0; u < EPT; ++u) xt[(e_row0 + u * kRowStep) * (kRowBytes / 2) + e_col] = cov[u];
          __syncthreads();
          const int64_t ntx = (p.xp_n + kTileN - 1) / kTileN;
          f32x16 xacc[MT][XPT];
#pragma unroll
          for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int i = 0; i < XPT; ++i)
#pragma unroll
              for (int r = 0; r < 16; ++r) xacc[mt][i][r] = 0.0f;
#pragma unroll
          for (int g = 0; g < XST; ++g)
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) {
              const u32x4 a = *reinterpret_cast<const u32x4*>(smem + mt * 32 * kRowBytes + rd_off + g * 32);
#pragma unroll
              for (int i = 0; i < XPT; ++i)
                if (wave + 4 * i < ntx) xacc[mt][i] = mfma<DT>(a, wx[i][g], xacc[mt][i]);
            }
          float* const dst = p.xp_part + t * p.M * p.xp_n;
#pragma unroll
          for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int i = 0; i < XPT; ++i)
#pragma unroll
              for (int r = 0; r < 16; ++r) {
                const int64_t m = 32 * mt + acc_row(r, lane);
                const int64_t n = 32 * (wave + 4 * i) + (lane & 31);
                if (m < p.M && n < p.xp_n) dst[m * p.xp_n + n] = xacc[mt][i][r];
              }
        }
      }
    }
  }
}

template <int DT, int KSW, int MT, int NT, int EPI, bool NORM = false, bool XP = false>
__global__ __launch_bounds__(KSW * 64) void linear_kernel(const LinParams p) {
  __shared__ __align__(16) char smem[LinLds<KSW, MT, NT, EPI>::kBytes];
  linear_body<DT, KSW, MT, NT, EPI, NORM, XP>(p, blockIdx.x, blockIdx.y, smem);
}

// in_proj + conv window + x_proj partials with the two halves on different column
// blocks: the conv half (n < n_conv), whose workgroups also run the conv step and the
// x_proj product after the K loop, on NTC = 1 tile (32 columns) per workgroup; the z half
// on NTZ = 2 tiles.  With the 2-tile blocks everywhere the conv-half workgroups (same
// weight and X bytes as the z half, plus the epilogue) set the kernel's time; on 1-tile
// blocks their K loop moves a third fewer bytes and the grid covers more CUs (Mamba-2.8B:
// 160 + 80 workgroups instead of 80 + 80).  Workgroups [0, conv_wgs) take the conv half.
template <int DT, int MT, int NTC, int NTZ>
__global__ __launch_bounds__(256) void in_proj_split_kernel(const LinParams p, int64_t conv_wgs) {
  constexpr int kC = LinLds<4, MT, NTC, MM_LIN_CONV>::kBytes;
  constexpr int kZ = LinLds<4, MT, NTZ, kZStore>::kBytes;
  __shared__ __align__(16) char smem[kC > kZ ? kC : kZ];
  const int64_t b = blockIdx.x;
  if (b < conv_wgs)
    linear_body<DT, 4, MT, NTC, MM_LIN_CONV, false, true>(p, b, 0, smem);
  else
    linear_body<DT, 4, MT, NTZ, kZStore>(p, p.n_conv / (NTZ * kTileN) + (b - conv_wgs), 0, smem);
}

// x_proj planes of mm_decode_in_proj_xproj summed: y[m, n] = round(sum_p part[p][m][n]).
// A workgroup covers 16 four-column groups; its 16 thread slices each sum a contiguous
// run of planes in order (all loads of a run issued together), then slice 0 adds the 16
// run sums in order -- a fixed summation order, so results are reproducible.  kRun (8 or
// 16, picked by the launcher) covers a slice's run in one round of loads up to 256
// planes.
template <int DT, int kRun>  // kRun: planes per thread slice and pass (loads in flight)
__global__ __launch_bounds__(256) void xp_reduce_kernel(const LinParams p, int64_t nplanes) {
  __shared__ f32x4 s_sum[16][16];
  const int gq = threadIdx.x & 15, sl = threadIdx.x >> 4;
  const int64_t nq = (p.xp_n + 3) / 4;
  const int64_t q = static_cast<int64_t>(blockIdx.x) * 16 + gq;
  const int64_t qc = q < p.M * nq ? q : 0;
  const int64_t m = qc / nq, n = (qc % nq) * 4;
  const int64_t plane = p.M * p.xp_n;
  const int64_t per = (nplanes + 15) / 16;
  const int64_t p0 = sl * per;
  const int64_t p1 = p0 + per < nplanes ? p0 + per : nplanes;
  f32x4 v = {0.0f, 0.0f, 0.0f, 0.0f};
  for (int64_t pb = p0; pb < p1; pb += kRun) {
    f32x4 a[kRun];
#pragma unroll
    for (int k = 0; k < kRun; ++k) {
      const int64_t pp = pb + k < p1 ? pb + k : p0;
      a[k] = *reinterpret_cast<const f32x4*>(p.xp_part + pp * plane + m * p.xp_n + n);
    }
#pragma unroll
    for (int k = 0; k < kRun; ++k)
      if (pb + k < p1) v += a[k];
  }
  s_sum[sl][gq] = v;
  __syncthreads();
  if (sl == 0 && q < p.M * nq) {
    f32x4 tot = s_sum[0][gq];
#pragma unroll
    for (int k = 1; k < 16; ++k) tot += s_sum[k][gq];
#pragma unroll
    for (int u = 0; u < 4; ++u)
      if (n + u < p.xp_n) st<DT>(p.xp_y, m * p.ld_xp + n + u, tot[u]);
  }
}

// a better than b for a greedy argmax: NaN first, then the larger value, then the lower
// index (torch.argmax's conventions, as mm_argmax_rows).
__device__ __forceinline__ bool arg_better(float av, int32_t ai, float bv, int32_t bi) {
  const bool an = av != av, bn = bv != bv;
  if (an != bn) return an;
  if (!an && av != bv) return av > bv;
  return ai < bi;
}

// mm_decode_head_argmax_embed: rows[m, :len] = table[ids[m], :len] (2-byte elements,
// len, both row strides multiple of 8 and 16-byte aligned rows: 8-element copies).
struct EmbedArgs {
  const u32x4* table;
  int64_t ld_table;
  u32x4* rows;
  int64_t ld_rows;
  int64_t len;
};

// The embedding row of id into row r, copied by the workgroup's 256 threads.
__device__ __forceinline__ void copy_embed_row(const EmbedArgs& e, int64_t r, int64_t id, int tid) {
  const u32x4* const src = e.table + id * (e.ld_table / 8);
  u32x4* const dst = e.rows + r * (e.ld_rows / 8);
  for (int64_t c = tid; c < e.len / 8; c += 256) dst[c] = src[c];
}

// Second pass of mm_decode_head_argmax: one workgroup per row picks among the nwg
// workgroup candidates (in that order, so ties keep the lowest column); with an
// embedding table (e.table) it then writes the chosen id's embedding row.
__global__ __launch_bounds__(256) void head_argmax_kernel(const float* __restrict__ cand_v,
                                                          const int32_t* __restrict__ cand_i,
                                                          int64_t nwg, int64_t M,
                                                          int64_t* __restrict__ ids,
                                                          const EmbedArgs e) {
  __shared__ float s_v[4];
  __shared__ int32_t s_i[4];
  __shared__ int32_t s_id;
  const int64_t r = blockIdx.x;
  const int tid = threadIdx.x;
  float bv = -__builtin_inff();
  int32_t bi = 0x7fffffff;
  for (int64_t w = tid; w < nwg; w += 256) {
    const float v = cand_v[w * M + r];
    const int32_t i = cand_i[w * M + r];
    if (arg_better(v, i, bv, bi)) {
      bv = v;
      bi = i;
    }
  }
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const float ov = lane_xor(bv, off);
    const int32_t oi = __float_as_int(lane_xor(__int_as_float(bi), off));
    if (arg_better(ov, oi, bv, bi)) {
      bv = ov;
      bi = oi;
    }
  }
  if ((tid & 63) == 0) {
    s_v[tid >> 6] = bv;
    s_i[tid >> 6] = bi;
  }
  __syncthreads();
  if (tid == 0) {
    bv = s_v[0];
    bi = s_i[0];
    for (int w = 1; w < 4; ++w)
      if (arg_better(s_v[w], s_i[w], bv, bi)) {
        bv = s_v[w];
        bi = s_i[w];
      }
    ids[r] = bi;
    s_id = bi;
  }
  if (e.table != nullptr) {
    __syncthreads();
    copy_embed_row(e, r, s_id, tid);
  }
}

// mm_decode_head_argmax_embed after a separate argmax (heads the fused path does not
// take): one workgroup per row copies the embedding row of ids[row].
__global__ __launch_bounds__(256) void embed_rows_kernel(const int64_t* __restrict__ ids,
                                                         const EmbedArgs e) {
  copy_embed_row(e, blockIdx.x, ids[blockIdx.x], threadIdx.x);
}

// Shared-X kernel for wide N.  Workgroup = NW waves; wave w owns the 32 columns
// n0 = (blockIdx.x * NW + w) * 32 and all of K.  Per 64-k chunk the waves load the
// X chunk together (8 rows per load instruction, instruction q by wave q % NW), write
// it to one of three LDS buffers and meet at a barrier; each wave then runs its 4 x MT
// MFMAs from that buffer.  W and X loads run two chunks ahead of the MFMAs through a
// three-slot register ring (named slots: an array indexed by slot would be moved to
// scratch or LDS).  A buffer is rewritten three chunks after it was read, i.e. after
// two more barriers, by which time every wave's reads of it have completed.  The
// epilogue stores straight from the accumulators: lane l holds column n0 + l % 32.
template <int XPW>
struct ShareSlot {
  u32x4 w[kSteps];
  u32x4 x[XPW];
};

template <int DT, int NW, int MT, int EPI>
__global__ __launch_bounds__(NW * 64, 1) void share_kernel(const LinParams p) {
  using T = typename Ty<DT>::T;
  constexpr int XQ = MT * 4;                  // X load instructions per chunk (8 rows each)
  constexpr int XPW = (XQ + NW - 1) / NW;     // per wave
  constexpr int kBuf = MT * 32 * kRowBytes;
  __shared__ __align__(16) char xs[3][kBuf];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int64_t n0 = (static_cast<int64_t>(blockIdx.x) * NW + wave) * kTileN;
  const int64_t nsteps = p.K / kStepK;
  // K range: all of K, or split blockIdx.y of gridDim.y (then the epilogue writes fp32
  // partials and the ordered reduce pass runs the real epilogue).  A range past the end
  // is empty: its loads re-read the last chunk and its partial tile is zero.
  const int64_t kch = p.K / kChunkK;
  const int64_t per_wg = (kch + gridDim.y - 1) / gridDim.y;
  const int64_t cbeg = static_cast<int64_t>(blockIdx.y) * per_wg;
  const int64_t nchunks = cbeg + per_wg < kch ? cbeg + per_wg : kch;  // end of this range
  const int64_t ntiles32 = (p.N + kTileN - 1) / kTileN;
  const int64_t tile = n0 / kTileN < ntiles32 ? n0 / kTileN : 0;
  const u32x4* const wp = static_cast<const u32x4*>(p.w) + tile * nsteps * 64 + lane;
  // X instruction q = wave + i * NW covers rows 8q .. 8q + 7 (lane: row 8q + l/8,
  // 16-byte column l % 8).  Slots past XQ re-load a valid row and are not stored.
  const T* xrow[XPW];
  bool xok[XPW];
#pragma unroll
  for (int i = 0; i < XPW; ++i) {
    const int q = wave + i * NW;
    xok[i] = q < XQ;
    const int64_t r = 8 * (q < XQ ? q : 0) + (lane >> 3);
    xrow[i] = static_cast<const T*>(p.x) + (r < p.M ? r : 0) * p.ldx + 8 * (lane & 7);
  }
  const int rd_off = (lane & 31) * kRowBytes + (lane >> 5) * 16;

  // The conv epilogue's inputs do not depend on the product: load them before the
  // K loop so their latency hides under it (clamped: lanes past n_conv read column 0).
  typedef T T4 __attribute__((ext_vector_type(4)));
  const int64_t n = n0 + (lane & 31);
  const bool ncol = n < p.N;
  T4 win[EPI == MM_LIN_CONV ? MT : 1][16];
  T4 cw{};
  float bias = 0.0f;
  if constexpr (EPI == MM_LIN_CONV) {
    const int64_t nc = n < p.n_conv ? n : 0;
    const T4* const sb = static_cast<const T4*>(p.conv_state);
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int64_t m = 32 * mt + acc_row(i, lane);
        win[mt][i] = sb[(m < p.M ? m : 0) * p.n_conv + nc];
      }
    cw = static_cast<const T4*>(p.conv_w)[nc];
    const T* const bb = static_cast<const T*>(p.conv_b ? p.conv_b : p.conv_w);
    bias = p.conv_b ? Ty<DT>::f(bb[nc]) : 0.0f;
  }

  f32x16 acc[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[mt][i] = 0.0f;

  using S = ShareSlot<XPW>;
  const int64_t clast = nchunks - 1;
  auto load = [&](S& s, int64_t c) __attribute__((always_inline)) {
    const int64_t cc = c < nchunks ? c : clast;
#pragma unroll
    for (int g = 0; g < kSteps; ++g) s.w[g] = wp[(cc * kSteps + g) * 64];
#pragma unroll
    for (int i = 0; i < XPW; ++i) s.x[i] = *reinterpret_cast<const u32x4*>(xrow[i] + cc * kChunkK);
  };
  auto compute = [&](S& s, int64_t c, int buf) __attribute__((always_inline)) {
    if (c >= nchunks) return;  // uniform over the workgroup
    char* const xb = xs[buf];
#pragma unroll
    for (int i = 0; i < XPW; ++i)
      if (XQ % NW == 0 || xok[i])
        *reinterpret_cast<u32x4*>(xb + (8 * (wave + i * NW) + (lane >> 3)) * kRowBytes + (lane & 7) * 16) = s.x[i];
    __syncthreads();
#pragma unroll
    for (int g = 0; g < kSteps; ++g)
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        const u32x4 a = *reinterpret_cast<const u32x4*>(xb + mt * 32 * kRowBytes + rd_off + g * 32);
        acc[mt] = mfma<DT>(a, s.w[g], acc[mt]);
      }
  };
  S s0, s1, s2;
  load(s0, cbeg);
  load(s1, cbeg + 1);
  // Whole rounds while all three prefetches stay in range, then the last 1-4 chunks
  // straight-line: the round's prefetches of c + 3 and c + 4 would otherwise re-read
  // the last chunk up to four more times.  The conv epilogue keeps the plain loop: with
  // its registers live the peeled tail would spill.
  int64_t c = cbeg;
  if constexpr (EPI == MM_LIN_CONV) {
    for (; c < nchunks; c += 3) {
      load(s2, c + 2);
      compute(s0, c, 0);
      load(s0, c + 3);
      compute(s1, c + 1, 1);
      load(s1, c + 4);
      compute(s2, c + 2, 2);
    }
    c = nchunks;  // nothing left for the tail below
  }
  for (; c + 4 < nchunks; c += 3) {
    load(s2, c + 2);
    compute(s0, c, 0);
    load(s0, c + 3);
    compute(s1, c + 1, 1);
    load(s1, c + 4);
    compute(s2, c + 2, 2);
  }
  switch (nchunks - c) {  // uniform over the workgroup
    case 4:
      load(s2, c + 2);
      compute(s0, c, 0);
      load(s0, c + 3);
      compute(s1, c + 1, 1);
      compute(s2, c + 2, 2);
      compute(s0, c + 3, 0);
      break;
    case 3:
      load(s2, c + 2);
      compute(s0, c, 0);
      compute(s1, c + 1, 1);
      compute(s2, c + 2, 2);
      break;
    case 2:
      compute(s0, c, 0);
      compute(s1, c + 1, 1);
      break;
    default:
      compute(s0, c, 0);
      break;
  }

  // ---- epilogue: lane holds column n0 + l % 32, rows 32 mt + acc_row(i, l) ----
  if constexpr (EPI == kPartial) {
    float* const dst = p.partials + static_cast<int64_t>(blockIdx.y) * p.M * p.N;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int64_t m = 32 * mt + acc_row(i, lane);
        if (ncol && m < p.M) dst[m * p.N + n] = acc[mt][i];
      }
  } else if constexpr (EPI == MM_LIN_STORE || EPI == kStoreArgmax) {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int64_t m = 32 * mt + acc_row(i, lane);
        if (ncol && m < p.M) st<DT>(p.y, m * p.ldy + n, acc[mt][i]);
      }
    if constexpr (EPI == kStoreArgmax) {
      // Greedy argmax of the stored (rounded) logits, torch.argmax's order: NaN first,
      // then the larger value, then the lower column.  Per m-tile each wave transposes its
      // 32 x 32 tile through LDS (lane l holds rows acc_row(., l) of column l % 32); lane
      // l then scans row l / 2, columns 16 (l % 2) .. + 15 in order, the two halves meet
      // in one exchange, and the NW waves' row maxima are combined in wave order (lower
      // columns first).  One candidate per row and workgroup goes to cand_v / cand_i;
      // head_argmax_kernel picks among those.
      __shared__ float s_t[NW][32][33];
      __syncthreads();  // every wave is past its last MFMA read of xs
      float* const cv = reinterpret_cast<float*>(&xs[0][0]);      // [NW][MT * 32]
      int32_t* const ci = reinterpret_cast<int32_t*>(cv + NW * MT * 32);
      const int r = lane >> 1, half = lane & 1;
      const int64_t nw0 = n0;  // this wave's first column
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
        for (int i = 0; i < 16; ++i)
          s_t[wave][acc_row(i, lane)][lane & 31] =
              ncol ? Ty<DT>::f(Ty<DT>::from(acc[mt][i])) : -__builtin_inff();
        __builtin_amdgcn_wave_barrier();  // LDS is in order per wave: the reads see the writes
        float bv = -__builtin_inff();
        int32_t bi = 0x7fffffff;
        if (32 * mt + r < p.M) {
#pragma unroll
          for (int c = 0; c < 16; ++c) {
            const int col = 16 * half + c;
            const float v = s_t[wave][r][col];
            const bool in = nw0 + col < p.N;
            const bool t = in && (bi == 0x7fffffff || v > bv || (v != v && bv == bv));
            bv = t ? v : bv;
            bi = t ? static_cast<int32_t>(nw0 + col) : bi;
          }
        }
        const float ov = lane_xor(bv, 1);
        const int32_t oi = __float_as_int(lane_xor(__int_as_float(bi), 1));
        if (arg_better(ov, oi, bv, bi)) {
          bv = ov;
          bi = oi;
        }
        if (half == 0) {
          cv[wave * MT * 32 + 32 * mt + r] = bv;
          ci[wave * MT * 32 + 32 * mt + r] = bi;
        }
        __builtin_amdgcn_wave_barrier();  // the next m-tile rewrites s_t[wave]
      }
      __syncthreads();
      if (threadIdx.x < MT * 32 && threadIdx.x < p.M) {
        const int rr = threadIdx.x;
        float bv = cv[rr];
        int32_t bi = ci[rr];
#pragma unroll
        for (int w = 1; w < NW; ++w)
          if (arg_better(cv[w * MT * 32 + rr], ci[w * MT * 32 + rr], bv, bi)) {
            bv = cv[w * MT * 32 + rr];
            bi = ci[w * MT * 32 + rr];
          }
        p.cand_v[static_cast<int64_t>(blockIdx.x) * p.M + rr] = bv;
        p.cand_i[static_cast<int64_t>(blockIdx.x) * p.M + rr] = bi;
      }
    }
  } else if constexpr (EPI == MM_LIN_RESID) {
    T* const rb = static_cast<T*>(p.resid);
    T old[MT][16];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int64_t m = 32 * mt + acc_row(i, lane);
        old[mt][i] = rb[(ncol && m < p.M) ? m * p.ldr + n : 0];
      }
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int64_t m = 32 * mt + acc_row(i, lane);
        if (ncol && m < p.M)
          rb[m * p.ldr + n] = Ty<DT>::from(Ty<DT>::f(old[mt][i]) + Ty<DT>::f(Ty<DT>::from(acc[mt][i])));
      }
  } else {
    if (n < p.n_conv) {
      T4* const sb = static_cast<T4*>(p.conv_state);
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int64_t m = 32 * mt + acc_row(i, lane);
          if (m >= p.M) continue;
          const T xr = Ty<DT>::from(acc[mt][i]);
          float a = bias;
          a = __builtin_fmaf(Ty<DT>::f(cw[0]), Ty<DT>::f(win[mt][i][1]), a);
          a = __builtin_fmaf(Ty<DT>::f(cw[1]), Ty<DT>::f(win[mt][i][2]), a);
          a = __builtin_fmaf(Ty<DT>::f(cw[2]), Ty<DT>::f(win[mt][i][3]), a);
          a = __builtin_fmaf(Ty<DT>::f(cw[3]), Ty<DT>::f(xr), a);
          T4 nw;
          nw[0] = win[mt][i][1];
          nw[1] = win[mt][i][2];
          nw[2] = win[mt][i][3];
          nw[3] = xr;
          sb[m * p.n_conv + n] = nw;
          st<DT>(p.conv_out, m * p.ldc + n, silu_f(a));
        }
    } else if (ncol) {
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int64_t m = 32 * mt + acc_row(i, lane);
          if (m < p.M) st<DT>(p.y, m * p.ldy + (n - p.n_conv), acc[mt][i]);
        }
    }
  }
}

// Split calls, second pass: y = sum over splits (in order) of the fp32 partials,
// then the epilogue.  One thread per 4 consecutive columns of a row; the KS loads
// of a thread are all issued before the sum (KS is a template parameter).
template <int DT, int EPI, int KS>
__global__ __launch_bounds__(256) void reduce_kernel(const LinParams p) {
  const int64_t q = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  const int64_t nq = (p.N + 3) / 4;
  if (q >= p.M * nq) return;
  const int64_t m = q / nq, n = (q % nq) * 4;
  const int64_t plane = p.M * p.N;
  const float* src = p.partials + m * p.N + n;
  float v[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  if (n + 4 <= p.N && (p.N & 3) == 0) {
    f32x4 a[KS];
#pragma unroll
    for (int k = 0; k < KS; ++k) a[k] = *reinterpret_cast<const f32x4*>(src + k * plane);
#pragma unroll
    for (int k = 0; k < KS; ++k) {
      v[0] += a[k][0];
      v[1] += a[k][1];
      v[2] += a[k][2];
      v[3] += a[k][3];
    }
  } else {
    for (int k = 0; k < KS; ++k)
      for (int u = 0; u < 4; ++u)
        if (n + u < p.N) v[u] += src[k * plane + u];
  }
  for (int u = 0; u < 4; ++u)
    if (n + u < p.N) epilogue<DT, EPI>(p, m, n + u, v[u]);
}

// Split calls with MM_LIN_RESID_NORM, second pass: one workgroup per row sums the
// splits (in order), updates the residual row and writes its RMSNorm.  Thread t
// takes float4 column groups t, t + 256, ...; all loads (partials, residual, norm
// weight) are issued before the first sum.
template <int DT, int KS, int CPT>
__global__ __launch_bounds__(256) void reduce_norm_kernel(const LinParams p) {
  using T = typename Ty<DT>::T;
  typedef T T4 __attribute__((ext_vector_type(4)));
  __shared__ float s_part[4];
  const int64_t m = blockIdx.x;
  const int tid = threadIdx.x;
  const int64_t ng = p.N / 4;
  const int64_t plane = p.M * p.N;
  T4* const rrow = reinterpret_cast<T4*>(static_cast<T*>(p.resid) + m * p.ldr);
  const T4* const wrow = static_cast<const T4*>(p.norm_w);
  f32x4 part[CPT][KS];
  T4 rv[CPT], wv[CPT];
#pragma unroll
  for (int u = 0; u < CPT; ++u) {
    const int64_t g = tid + 256 * u < ng ? tid + 256 * u : 0;
#pragma unroll
    for (int k = 0; k < KS; ++k)
      part[u][k] = *reinterpret_cast<const f32x4*>(p.partials + k * plane + m * p.N + 4 * g);
    rv[u] = rrow[g];
    wv[u] = wrow[g];
  }
  float nv[CPT][4];
  float ss = 0.0f;
#pragma unroll
  for (int u = 0; u < CPT; ++u) {
    const bool ok = tid + 256 * u < ng;
    T4 o;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      float a = 0.0f;
#pragma unroll
      for (int k = 0; k < KS; ++k) a += part[u][k][e];
      const T r = Ty<DT>::from(Ty<DT>::f(rv[u][e]) + Ty<DT>::f(Ty<DT>::from(a)));
      o[e] = r;
      nv[u][e] = ok ? Ty<DT>::f(r) : 0.0f;
      ss = __builtin_fmaf(nv[u][e], nv[u][e], ss);
    }
    if (ok) rrow[tid + 256 * u] = o;
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) ss += lane_xor(ss, off);
  if ((tid & 63) == 0) s_part[tid >> 6] = ss;
  __syncthreads();
  const float inv = rsqrtf((s_part[0] + s_part[1] + s_part[2] + s_part[3]) / static_cast<float>(p.N) + p.eps);
  T4* const orow = reinterpret_cast<T4*>(static_cast<T*>(p.norm_out) + m * p.ldn);
#pragma unroll
  for (int u = 0; u < CPT; ++u) {
    if (tid + 256 * u < ng) {
      T4 o;
#pragma unroll
      for (int e = 0; e < 4; ++e) o[e] = norm_round<DT>(nv[u][e], inv, Ty<DT>::f(wv[u][e]));
      orow[tid + 256 * u] = o;
    }
  }
}

// Small-M path (M <= 4): a weight-streaming GEMV.  With one to four rows the 32-row
// MFMA tile is mostly padding and the kernel is pure weight streaming, whose rate is set
// per CU (an L1 keeps ~84 L2 reads of 128 bytes in flight, ~40 GB/s): what matters is
// spreading W evenly over all CUs.  A workgroup owns 8 output columns and all of K.
// Thread t takes column n0 + t%8, half (t/8)%2 of each 16-wide k step, and steps
// t/16, t/16 + SG, ... (SG = NT / 16 step groups): in the packed layout each 16-thread
// group reads two contiguous 128-byte pieces per step.  Each thread accumulates in k
// order in fp32; the NT / 8 threads of a column are combined by an xor-shuffle tree
// (within a wave) and then in wave order through LDS -- deterministic.  Loads are issued
// U steps at a time ahead of their use (clamped to the last step: every load is in bounds
// and unconditional, and a clamped step is multiplied in with a zero weight).  The
// workgroup size NT (256, 512 or 1024, at most 1024 / rows) gives each thread at most 4
// steps, so one load round covers K (a dependent memory round trip per further round is
// what this latency-bound kernel pays for), and U (3 or 4) is then picked from the steps
// per thread:
// fewest rounds, then fewest clamped steps.  Measured at the Mamba-130M decode (K = 768
// and 1536): U = 3 instead of 4 wastes no step (0.370-0.382 -> 0.364 ms per step; U = 2,
// 6, 8 measured 0.40, 0.39, 0.42 ms), and 512 threads for K = 1536 take x_proj and
// out_proj from two load rounds to one (0.355 -> 0.337 ms per step).  The input
// RMSNorm (NORM) is computed by wave 0 in add_rmsnorm_vec_kernel's order and applied as
// each x chunk is loaded, as in linear_kernel.  Epilogues as the split-K reduce.
constexpr int kGvCols = 8;
constexpr int kGvMaxM = 4;

template <int DT, int MM, int EPI, bool NORM, int U, int NT>
__global__ __launch_bounds__(NT) void gemv_kernel(const LinParams p) {
  constexpr int SG = NT / 16;  // step groups: thread t walks steps t/16, t/16 + SG, ...
  using T = typename Ty<DT>::T;
  using V8 = typename Ty<DT>::V8;
  __shared__ float s_red[NT / 64][MM][kGvCols];
  __shared__ float s_inv[MM];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int j = tid & 7;
  const int hk = (tid >> 3) & 1;
  const int64_t n = static_cast<int64_t>(blockIdx.x) * kGvCols + j;
  const int64_t nc = n < p.N ? n : 0;
  const int64_t nsteps = p.K / kStepK;
  const u32x4* const wb = static_cast<const u32x4*>(p.w) + (nc >> 5) * nsteps * 64 + (nc & 31) + 32 * hk;
  const T* xr[MM];
#pragma unroll
  for (int m = 0; m < MM; ++m)
    xr[m] = static_cast<const T*>(p.x) + (m < p.M ? m : 0) * p.ldx + 8 * hk;

  // Load group at steps sb, sb + SG, ... (clamped to the last step; steps past the end
  // count with a zero weight when consumed).
  const int64_t s_last = nsteps - 1;
  u32x4 wv[U], nv[U];
  V8 xv[U][MM];
  auto load = [&](int64_t sb) __attribute__((always_inline)) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t st = sb + SG * u < nsteps ? sb + SG * u : s_last;
      wv[u] = wb[st * 64];
#pragma unroll
      for (int m = 0; m < MM; ++m) xv[u][m] = *reinterpret_cast<const V8*>(xr[m] + st * kStepK);
      if constexpr (NORM)
        nv[u] = *reinterpret_cast<const u32x4*>(static_cast<const T*>(p.x_norm_w) + st * kStepK + 8 * hk);
    }
  };
  int64_t sb = tid >> 4;
  load(sb);  // the first group's loads are in flight while the norm below runs

  if constexpr (NORM) {  // inverse RMS of each row, add_rmsnorm_vec_kernel's order
    if (wave == 0) {
      const int nch = static_cast<int>(p.K >> 3);
      for (int64_t m = 0; m < p.M; ++m) {
        const T* const r = static_cast<const T*>(p.x) + m * p.ldx;
        float ss = row_sumsq<DT>(r, nch, lane);
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) ss += lane_xor(ss, off);
        if (lane == 0) s_inv[m] = rsqrtf(ss / static_cast<float>(p.K) + p.x_eps);
      }
    }
    __syncthreads();
  }
  float xinv[MM];
#pragma unroll
  for (int m = 0; m < MM; ++m) xinv[m] = NORM ? s_inv[m < p.M ? m : 0] : 0.0f;

  float acc[MM];
#pragma unroll
  for (int m = 0; m < MM; ++m) acc[m] = 0.0f;
  for (;;) {
    // Consuming every loaded step (a zero weight past the end) keeps the compiler from
    // sinking the loads behind a branch.
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const u32x4 zero = {0u, 0u, 0u, 0u};
      const V8 w8 = __builtin_bit_cast(V8, sb + SG * u < nsteps ? wv[u] : zero);
#pragma unroll
      for (int m = 0; m < MM; ++m) {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          float x = Ty<DT>::f(xv[u][m][e]);
          if constexpr (NORM)
            x = Ty<DT>::f(norm_round<DT>(x, xinv[m], Ty<DT>::f(__builtin_bit_cast(V8, nv[u])[e])));
          acc[m] = __builtin_fmaf(x, Ty<DT>::f(w8[e]), acc[m]);
        }
      }
    }
    sb += SG * U;
    if (sb >= nsteps) break;
    load(sb);
  }
  // column sums: lanes j, j+8, ..., j+56 of a wave, then the NT / 64 waves in order
#pragma unroll
  for (int m = 0; m < MM; ++m) {
#pragma unroll
    for (int off = 8; off < 64; off <<= 1) acc[m] += lane_xor(acc[m], off);
    if (lane < kGvCols) s_red[wave][m][lane] = acc[m];
  }
  __syncthreads();
  if (tid < MM * kGvCols) {
    const int m = tid / kGvCols, jj = tid % kGvCols;
    const int64_t nn = static_cast<int64_t>(blockIdx.x) * kGvCols + jj;
    float v = s_red[0][m][jj];
#pragma unroll
    for (int w = 1; w < NT / 64; ++w) v += s_red[w][m][jj];
    if (m < p.M && nn < p.N) epilogue<DT, EPI>(p, m, nn, v);
  }
}

template <int DT, int MM, bool NORM, int U, int NT>
void launch_gemv_u(const LinParams& p, int32_t epi, hipStream_t s) {
  const dim3 grid(static_cast<unsigned>(ceil_div(p.N, kGvCols)));
  switch (epi) {
    case MM_LIN_STORE:
      hipLaunchKernelGGL((gemv_kernel<DT, MM, MM_LIN_STORE, NORM, U, NT>), grid, dim3(NT), 0, s, p);
      break;
    case MM_LIN_RESID:
      hipLaunchKernelGGL((gemv_kernel<DT, MM, MM_LIN_RESID, NORM, U, NT>), grid, dim3(NT), 0, s, p);
      break;
    default:
      hipLaunchKernelGGL((gemv_kernel<DT, MM, MM_LIN_CONV, NORM, U, NT>), grid, dim3(NT), 0, s, p);
      break;
  }
}

// Threads per workgroup: enough 16-thread step groups that each thread has at most 4 steps
// (one load round), up to 1024 / MM -- with more rows the per-thread registers (MM x-row
// vectors per step, the input-norm operands) no longer fit the smaller register share of a
// larger workgroup and would spill.
inline int gemv_threads(int64_t K, int mm) {
  const int64_t nsteps = K / kStepK;
  int nt = 256;
  while (nt < 1024 / mm && ceil_div(nsteps, nt / 16) > 4) nt *= 2;
  return nt;
}

// Steps loaded per round (see gemv_kernel): fewest rounds, then fewest clamped steps.
inline int gemv_group(int64_t K, int nt) {
  const int64_t t = ceil_div(K / kStepK, nt / 16);  // steps per thread
  const int64_t r3 = ceil_div(t, 3), r4 = ceil_div(t, 4);
  if (r4 < r3) return 4;
  return (r3 * 3 - t) < (r4 * 4 - t) ? 3 : 4;
}

template <int DT, int MM, bool NORM, int NT>
void launch_gemv_n(const LinParams& p, int32_t epi, hipStream_t s) {
  if (gemv_group(p.K, NT) == 3) launch_gemv_u<DT, MM, NORM, 3, NT>(p, epi, s);
  else launch_gemv_u<DT, MM, NORM, 4, NT>(p, epi, s);
}

template <int DT, int MM, bool NORM>
void launch_gemv_e(const LinParams& p, int32_t epi, hipStream_t s) {
  const int nt = gemv_threads(p.K, MM);
  if constexpr (MM == 1) {
    if (nt == 1024) return launch_gemv_n<DT, MM, NORM, 1024>(p, epi, s);
  }
  if constexpr (MM <= 2) {
    if (nt == 512) return launch_gemv_n<DT, MM, NORM, 512>(p, epi, s);
  }
  launch_gemv_n<DT, MM, NORM, 256>(p, epi, s);
}

template <int DT>
void launch_gemv(const LinParams& p, int32_t epi, hipStream_t s) {
  const bool norm = p.x_norm_w != nullptr;
#define MM_GV(MMV)                                       \
  if (norm) launch_gemv_e<DT, MMV, true>(p, epi, s);     \
  else launch_gemv_e<DT, MMV, false>(p, epi, s)
  if (p.M == 1) {
    MM_GV(1);
  } else if (p.M == 2) {
    MM_GV(2);
  } else {
    MM_GV(4);
  }
#undef MM_GV
}

// The GEMV covers M <= 4 where the shared-X kernel would not run (N <= 16384 columns).
inline bool use_gemv(int64_t M, int64_t N) {
  return M <= kGvMaxM && ceil_div(N, kTileN) <= kShareTiles;
}

// Packed layout: dst block (t, s), lane l = W[32t + l%32, 16s + 8(l/32) .. +7]
// (zero rows past N).  One thread per 16-byte piece.
template <int DT>
__global__ __launch_bounds__(256) void pack_kernel(const void* __restrict__ w, u32x4* __restrict__ dst,
                                                   int64_t N, int64_t K, int64_t ldw, int64_t total) {
  using T = typename Ty<DT>::T;
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i >= total) return;
  const int64_t nsteps = K / kStepK;
  const int lane = static_cast<int>(i & 63);
  const int64_t s = (i >> 6) % nsteps;
  const int64_t t = (i >> 6) / nsteps;
  const int64_t n = t * kTileN + (lane & 31);
  u32x4 v = {0u, 0u, 0u, 0u};
  if (n < N) v = *reinterpret_cast<const u32x4*>(static_cast<const T*>(w) + n * ldw + s * kStepK + 8 * (lane >> 5));
  dst[i] = v;
}

template <int DT, int KSW, int MT, int NT, bool NORM>
void launch_epi_n(const LinParams& p, int32_t epi, dim3 grid, hipStream_t s) {
  const dim3 block(KSW * 64);
  switch (epi) {
    case MM_LIN_STORE:
      hipLaunchKernelGGL((linear_kernel<DT, KSW, MT, NT, MM_LIN_STORE, NORM>), grid, block, 0, s, p);
      break;
    case MM_LIN_RESID:
      hipLaunchKernelGGL((linear_kernel<DT, KSW, MT, NT, MM_LIN_RESID, NORM>), grid, block, 0, s, p);
      break;
    case MM_LIN_CONV:
      hipLaunchKernelGGL((linear_kernel<DT, KSW, MT, NT, MM_LIN_CONV, NORM>), grid, block, 0, s, p);
      break;
    default:
      hipLaunchKernelGGL((linear_kernel<DT, 1, MT, NT, kPartial, NORM>), grid, dim3(64), 0, s, p);
      break;
  }
}

// The input-norm instantiations exist for one m-tile only (M <= 8, checked on the host).
template <int DT, int KSW, int MT, int NT>
void launch_epi(const LinParams& p, int32_t epi, dim3 grid, hipStream_t s) {
  if constexpr (MT == 1) {
    if (p.x_norm_w) {
      launch_epi_n<DT, KSW, MT, NT, true>(p, epi, grid, s);
      return;
    }
  }
  launch_epi_n<DT, KSW, MT, NT, false>(p, epi, grid, s);
}

template <int DT, int MT, int NT>
void launch_ksw(const LinParams& p, int32_t epi, int ksw, dim3 grid, hipStream_t s) {
  switch (ksw) {
    case 1: launch_epi<DT, 1, MT, NT>(p, epi, grid, s); break;
    case 2: launch_epi<DT, 2, MT, NT>(p, epi, grid, s); break;
    default: launch_epi<DT, 4, MT, NT>(p, epi, grid, s); break;
  }
}

template <int DT>
void launch_main(const LinParams& p, int32_t epi, const Plan& pl, dim3 grid, hipStream_t s) {
  const bool two = p.M > 32;
  if (two && pl.nt == 2) launch_ksw<DT, 2, 2>(p, epi, pl.ksw, grid, s);
  else if (two) launch_ksw<DT, 2, 1>(p, epi, pl.ksw, grid, s);
  else if (pl.nt == 2) launch_ksw<DT, 1, 2>(p, epi, pl.ksw, grid, s);
  else launch_ksw<DT, 1, 1>(p, epi, pl.ksw, grid, s);
}

// in_proj + conv window + x_proj partials (then xp_reduce_kernel): the 4-wave linear_kernel
// shapes only (see xp_fusable).
template <int DT>
void launch_xp_reduce(const LinParams& p, int64_t nplanes, hipStream_t s) {
  const dim3 rgrid(static_cast<unsigned>(ceil_div(p.M * ceil_div(p.xp_n, 4), 16)));
  if (ceil_div(nplanes, 16) > 8)
    hipLaunchKernelGGL((xp_reduce_kernel<DT, 16>), rgrid, dim3(256), 0, s, p, nplanes);
  else
    hipLaunchKernelGGL((xp_reduce_kernel<DT, 8>), rgrid, dim3(256), 0, s, p, nplanes);
}

// Whether in_proj_split_kernel runs the fused call: 2-tile column blocks in the plan, z
// blocks aligned to n_conv, and 1-tile conv blocks + 2-tile z blocks within one
// workgroup per CU.
inline bool xp_split(const LinParams& p, const Plan& pl) {
  const int64_t wgs = p.n_conv / kTileN + ceil_div(p.N - p.n_conv, 2 * kTileN);
  return pl.nt == 2 && p.n_conv % (2 * kTileN) == 0 && wgs <= num_cus();
}

template <int DT>
void launch_main_xp(const LinParams& p, const Plan& pl, dim3 grid, hipStream_t s) {
  const dim3 block(4 * 64);
  if (xp_split(p, pl)) {
    const int64_t conv_wgs = p.n_conv / kTileN;
    const dim3 sgrid(static_cast<unsigned>(conv_wgs + ceil_div(p.N - p.n_conv, 2 * kTileN)));
    if (p.M > 32)
      hipLaunchKernelGGL((in_proj_split_kernel<DT, 2, 1, 2>), sgrid, block, 0, s, p, conv_wgs);
    else
      hipLaunchKernelGGL((in_proj_split_kernel<DT, 1, 1, 2>), sgrid, block, 0, s, p, conv_wgs);
    launch_xp_reduce<DT>(p, conv_wgs, s);
    return;
  }
  if (p.M > 32 && pl.nt == 2)
    hipLaunchKernelGGL((linear_kernel<DT, 4, 2, 2, MM_LIN_CONV, false, true>), grid, block, 0, s, p);
  else if (p.M > 32)
    hipLaunchKernelGGL((linear_kernel<DT, 4, 2, 1, MM_LIN_CONV, false, true>), grid, block, 0, s, p);
  else if (pl.nt == 2)
    hipLaunchKernelGGL((linear_kernel<DT, 4, 1, 2, MM_LIN_CONV, false, true>), grid, block, 0, s, p);
  else
    hipLaunchKernelGGL((linear_kernel<DT, 4, 1, 1, MM_LIN_CONV, false, true>), grid, block, 0, s, p);
  launch_xp_reduce<DT>(p, p.n_conv / (kTileN * pl.nt), s);
}

// Whether mm_decode_in_proj_xproj folds x_proj into in_proj's conv epilogue: the call
// must run linear_kernel with K in the workgroup over 4 waves (no GEMV, no shared-X
// kernel, no K split, no input RMSNorm), every workgroup's columns must lie on one side
// of n_conv, and x_proj must have at most 8 column tiles, a multiple of 4 columns.
inline bool xp_fusable(int64_t M, int64_t N, int64_t K, int64_t n_conv, int64_t xp_n, bool x_norm) {
  if (x_norm || M < 1 || M > kMaxM || N < 1 || K % kChunkK != 0 || use_gemv(M, N)) return false;
  const Plan pl = plan(N, K);
  if (pl.nw > 0 || pl.ks != 1 || pl.ksw != 4) return false;
  const int64_t tn = kTileN * pl.nt;
  return xp_n >= 4 && xp_n <= 8 * kTileN && xp_n % 4 == 0 && n_conv >= tn && n_conv % tn == 0 &&
         n_conv % kChunkK == 0;
}

// One fp32 (M, xp_n) plane per conv-half workgroup; sized for 1-tile conv blocks (the
// split kernel's, the larger count) whatever the device, so the size does not depend on it.
inline size_t xp_workspace(int64_t M, int64_t N, int64_t K, int64_t n_conv, int64_t xp_n) {
  (void)N;
  (void)K;
  return static_cast<size_t>(n_conv / kTileN) * static_cast<size_t>(M * xp_n) * 4;
}

struct XpArgs {
  const void* w;
  int64_t n;
  void* y;
  int64_t ld;
};

template <int DT, int NW, int MT>
void launch_share_epi(const LinParams& p, int32_t epi, dim3 grid, hipStream_t s) {
  const dim3 block(NW * 64);
  switch (epi) {
    case kPartial:
      hipLaunchKernelGGL((share_kernel<DT, NW, MT, kPartial>), grid, block, 0, s, p);
      break;
    case MM_LIN_STORE:
      hipLaunchKernelGGL((share_kernel<DT, NW, MT, MM_LIN_STORE>), grid, block, 0, s, p);
      break;
    case MM_LIN_RESID:
      hipLaunchKernelGGL((share_kernel<DT, NW, MT, MM_LIN_RESID>), grid, block, 0, s, p);
      break;
    case kStoreArgmax:
      hipLaunchKernelGGL((share_kernel<DT, NW, MT, kStoreArgmax>), grid, block, 0, s, p);
      break;
    default:
      hipLaunchKernelGGL((share_kernel<DT, NW, MT, MM_LIN_CONV>), grid, block, 0, s, p);
      break;
  }
}

template <int DT, int MT>
void launch_share_nw(const LinParams& p, int32_t epi, int nw, dim3 grid, hipStream_t s) {
  if (nw == 4) launch_share_epi<DT, 4, MT>(p, epi, grid, s);
  else launch_share_epi<DT, 8, MT>(p, epi, grid, s);
}

template <int DT>
void launch_share(const LinParams& p, int32_t epi, const Plan& pl, dim3 grid, hipStream_t s) {
  if (p.M > 32) launch_share_nw<DT, 2>(p, epi, pl.nw, grid, s);
  else launch_share_nw<DT, 1>(p, epi, pl.nw, grid, s);
}

template <int DT, int EPI>
void launch_reduce_ks(const LinParams& p, dim3 grid, hipStream_t s) {
  switch (p.ks) {
    case 2: hipLaunchKernelGGL((reduce_kernel<DT, EPI, 2>), grid, dim3(256), 0, s, p); break;
    case 4: hipLaunchKernelGGL((reduce_kernel<DT, EPI, 4>), grid, dim3(256), 0, s, p); break;
    case 8: hipLaunchKernelGGL((reduce_kernel<DT, EPI, 8>), grid, dim3(256), 0, s, p); break;
    case 16: hipLaunchKernelGGL((reduce_kernel<DT, EPI, 16>), grid, dim3(256), 0, s, p); break;
    case 32: hipLaunchKernelGGL((reduce_kernel<DT, EPI, 32>), grid, dim3(256), 0, s, p); break;
    default: hipLaunchKernelGGL((reduce_kernel<DT, EPI, 64>), grid, dim3(256), 0, s, p); break;
  }
}

template <int DT>
void launch_reduce(const LinParams& p, int32_t epi, hipStream_t s) {
  const dim3 grid(static_cast<unsigned>(ceil_div(p.M * ceil_div(p.N, 4), 256)));
  switch (epi) {
    case MM_LIN_STORE: launch_reduce_ks<DT, MM_LIN_STORE>(p, grid, s); break;
    case MM_LIN_RESID: launch_reduce_ks<DT, MM_LIN_RESID>(p, grid, s); break;
    default: launch_reduce_ks<DT, MM_LIN_CONV>(p, grid, s); break;
  }
}

template <int DT, int KS>
void launch_reduce_norm_ks(const LinParams& p, hipStream_t s) {
  const dim3 grid(static_cast<unsigned>(p.M));
  const int64_t ng = p.N / 4;
  if (ng <= 256) hipLaunchKernelGGL((reduce_norm_kernel<DT, KS, 1>), grid, dim3(256), 0, s, p);
  else if (ng <= 512) hipLaunchKernelGGL((reduce_norm_kernel<DT, KS, 2>), grid, dim3(256), 0, s, p);
  else hipLaunchKernelGGL((reduce_norm_kernel<DT, KS, 4>), grid, dim3(256), 0, s, p);
}

template <int DT>
void launch_reduce_norm(const LinParams& p, hipStream_t s) {
  switch (p.ks) {
    case 2: launch_reduce_norm_ks<DT, 2>(p, s); break;
    case 4: launch_reduce_norm_ks<DT, 4>(p, s); break;
    case 8: launch_reduce_norm_ks<DT, 8>(p, s); break;
    default: launch_reduce_norm_ks<DT, 16>(p, s); break;
  }
}

// The fused reduce + residual + RMSNorm pass covers split calls with <= 16 splits,
// N % 4 == 0, N <= 4096 and 8-byte aligned rows; otherwise the RESID epilogue runs
// and the norm follows as mm_add_rmsnorm.
inline bool fused_norm_ok(const LinParams& p, int32_t dtype, const void* resid, const void* norm_w,
                          const void* norm_out) {
  const int64_t vb = 4 * dtype_size(dtype);
  return p.ks > 1 && p.ks <= 16 && p.N % 4 == 0 && p.N <= 4096 && aligned(resid, vb) &&
         aligned(norm_w, vb) && aligned(norm_out, vb) && (p.ldr * dtype_size(dtype)) % vb == 0 &&
         (p.ldn * dtype_size(dtype)) % vb == 0;
}

}  // namespace gemm
}  // namespace mm

extern "C" {

size_t mm_packed_linear_weight_bytes(int64_t N, int64_t K, int32_t dtype) {
  using namespace mm;
  if (N <= 0 || K <= 0 || !valid_dtype(dtype)) return 0;
  return static_cast<size_t>(round_up(N, gemm::kTileN) * K * dtype_size(dtype));
}

int mm_pack_linear_weight(const void* w, void* packed, int64_t N, int64_t K, int64_t ldw,
                          int32_t dtype, void* stream) {
  using namespace mm;
  using namespace mm::gemm;
  clear_error();
  if (!w || !packed) return fail(MM_ERR_NULL_POINTER, "w and packed are required");
  if (N < 0 || K < 0) return fail(MM_ERR_SHAPE, "negative size");
  if (dtype != MM_F16 && dtype != MM_BF16) return fail(MM_ERR_DTYPE, "dtype must be f16 or bf16");
  if (K % kChunkK != 0 || ldw < K || ldw % 8 != 0 || !aligned(w, 16) || !aligned(packed, 16))
    return fail(MM_ERR_LAYOUT, "K must be a multiple of %d, ldw >= K a multiple of 8, "
                "w and packed 16-byte aligned", kChunkK);
  if (N == 0 || K == 0) return MM_OK;
  const int64_t total = ceil_div(N, kTileN) * (K / kStepK) * 64;
  const dim3 grid(static_cast<unsigned>(ceil_div(total, 256)));
  hipStream_t s = static_cast<hipStream_t>(stream);
  u32x4* dst = static_cast<u32x4*>(packed);
  if (dtype == MM_F16)
    hipLaunchKernelGGL((pack_kernel<MM_F16>), grid, dim3(256), 0, s, w, dst, N, K, ldw, total);
  else
    hipLaunchKernelGGL((pack_kernel<MM_BF16>), grid, dim3(256), 0, s, w, dst, N, K, ldw, total);
  return check_launch("pack_linear_weight");
}

size_t mm_decode_linear_workspace_size(int64_t M, int64_t N, int64_t K) {
  using namespace mm;
  using namespace mm::gemm;
  if (M <= 0 || N <= 0 || K <= 0 || M > kMaxM || K % kChunkK != 0) return 0;
  if (use_gemv(M, N)) return 0;
  const Plan pl = plan(N, K);
  if (pl.ks == 1) return 0;
  return static_cast<size_t>(pl.ks * M * N * 4);
}

}  // extern "C"

namespace mm {
namespace gemm {

// mm_decode_linear; with xp (only when xp_fusable) in_proj's conv epilogue also runs
// x_proj on the conv outputs.
// Whether mm_decode_head_argmax takes the argmax candidates in the GEMM's epilogue: the
// shared-X kernel without a K split (the LM head's wide N) and a plain store.
inline bool head_fusable(int64_t M, int64_t N, int64_t K) {
  if (M < 1 || M > kMaxM || N < 1 || K < 1 || K % kChunkK != 0 || use_gemv(M, N)) return false;
  const Plan pl = plan(N, K);
  return pl.nw > 0 && pl.ks == 1;
}

inline size_t head_cand_bytes(int64_t M, int64_t N, int64_t K) {
  const Plan pl = plan(N, K);
  return static_cast<size_t>(ceil_div(N, kTileN * pl.nw)) * static_cast<size_t>(M) * 8;
}

static int decode_linear_core(const mm_linear_params* prm, void* stream, const XpArgs* xp,
                              int64_t* argmax_ids = nullptr, const EmbedArgs* embed = nullptr) {
  if (!prm) return fail(MM_ERR_NULL_POINTER, "params is NULL");
  const mm_linear_params& q = *prm;
  if (!q.x || !q.w_packed) return fail(MM_ERR_NULL_POINTER, "x and w_packed are required");
  if (q.M < 0 || q.N < 0 || q.K < 0) return fail(MM_ERR_SHAPE, "negative size");
  if (q.M > kMaxM) return fail(MM_ERR_SHAPE, "M=%lld exceeds %d", (long long)q.M, kMaxM);
  if (q.dtype != MM_F16 && q.dtype != MM_BF16)
    return fail(MM_ERR_DTYPE, "dtype %d: the decode GEMM takes f16 or bf16", q.dtype);
  if (q.epilogue != MM_LIN_STORE && q.epilogue != MM_LIN_RESID && q.epilogue != MM_LIN_CONV &&
      q.epilogue != MM_LIN_RESID_NORM)
    return fail(MM_ERR_SHAPE, "unknown epilogue %d", q.epilogue);
  if (q.K % kChunkK != 0 || q.ldx < q.K || q.ldx % 8 != 0 || !aligned(q.x, 16) ||
      !aligned(q.w_packed, 16))
    return fail(MM_ERR_LAYOUT, "K must be a multiple of %d, ldx >= K a multiple of 8, x and "
                "w_packed 16-byte aligned", kChunkK);
  if (q.N > 0x7fffffffLL) return fail(MM_ERR_SHAPE, "N too large");
  if (q.epilogue == MM_LIN_STORE && !q.y) return fail(MM_ERR_NULL_POINTER, "y is required");
  if ((q.epilogue == MM_LIN_RESID || q.epilogue == MM_LIN_RESID_NORM) && !q.resid)
    return fail(MM_ERR_NULL_POINTER, "resid is required");
  if (q.epilogue == MM_LIN_RESID_NORM) {
    if (!q.norm_w || !q.norm_out) return fail(MM_ERR_NULL_POINTER, "norm_w and norm_out are required");
    if (!(q.eps >= 0.0f)) return fail(MM_ERR_SHAPE, "eps must be >= 0");
  }
  if (q.epilogue == MM_LIN_CONV) {
    if (!q.conv_state || !q.conv_w || !q.conv_out || (!q.y && q.n_conv < q.N))
      return fail(MM_ERR_NULL_POINTER, "conv_state, conv_w, conv_out and y are required");
    if (q.n_conv < 0 || q.n_conv > q.N) return fail(MM_ERR_SHAPE, "n_conv outside [0, N]");
    if (!aligned(q.conv_state, 8) || !aligned(q.conv_w, 8))
      return fail(MM_ERR_LAYOUT, "conv_state and conv_w must be 8-byte aligned");
  }
  if (q.reserved != 0) return fail(MM_ERR_LAYOUT, "reserved field must be 0");
  if (q.x_norm_w) {
    if (q.M > kNormInMaxM)
      return fail(MM_ERR_SHAPE, "the input RMSNorm takes M <= %d (M=%lld)", kNormInMaxM, (long long)q.M);
    if (q.K > kNormInMaxK)
      return fail(MM_ERR_SHAPE, "the input RMSNorm takes K <= %d", kNormInMaxK);
    if (ceil_div(q.N, kTileN) > kShareTiles)
      return fail(MM_ERR_SHAPE, "the input RMSNorm takes N <= %d", kShareTiles * kTileN);
    if (!aligned(q.x_norm_w, 16)) return fail(MM_ERR_LAYOUT, "x_norm_w must be 16-byte aligned");
    if (!(q.x_eps >= 0.0f)) return fail(MM_ERR_SHAPE, "x_eps must be >= 0");
  }
  if (q.M == 0 || q.N == 0) return MM_OK;
  const Plan pl = plan(q.N, q.K);
  const bool fuse_argmax = argmax_ids != nullptr && q.epilogue == MM_LIN_STORE && !q.x_norm_w &&
                           head_fusable(q.M, q.N, q.K);
  size_t need = xp ? xp_workspace(q.M, q.N, q.K, q.n_conv, xp->n)
                   : mm_decode_linear_workspace_size(q.M, q.N, q.K);
  if (fuse_argmax) need = std::max(need, head_cand_bytes(q.M, q.N, q.K));
  if (need > 0) {
    if (!q.workspace || q.workspace_bytes < need)
      return fail(MM_ERR_WORKSPACE, "workspace of %zu bytes required (got %zu)", need,
                  q.workspace ? q.workspace_bytes : (size_t)0);
    if (!aligned(q.workspace, 16)) return fail(MM_ERR_LAYOUT, "workspace must be 16-byte aligned");
  }
  LinParams p;
  p.x = q.x;
  p.w = q.w_packed;
  p.y = q.y;
  p.resid = q.resid;
  p.conv_state = q.conv_state;
  p.conv_w = q.conv_w;
  p.conv_b = q.conv_b;
  p.conv_out = q.conv_out;
  p.norm_w = q.norm_w;
  p.norm_out = q.norm_out;
  p.ldn = q.ldn;
  p.eps = q.eps;
  p.partials = need ? static_cast<float*>(q.workspace) : nullptr;
  p.x_norm_w = q.x_norm_w;
  p.x_eps = q.x_eps;
  p.M = q.M;
  p.N = q.N;
  p.K = q.K;
  p.ldx = q.ldx;
  p.ldy = q.ldy;
  p.ldr = q.ldr;
  p.ldc = q.ldc;
  p.n_conv = q.n_conv;
  p.ks = use_gemv(q.M, q.N) ? 1 : pl.ks;  // the GEMV keeps K in the workgroup
  p.xp_w = xp ? static_cast<const u32x4*>(xp->w) : nullptr;
  p.xp_part = xp ? static_cast<float*>(q.workspace) : nullptr;
  p.xp_y = xp ? xp->y : nullptr;
  p.xp_n = xp ? xp->n : 0;
  p.xp_nsteps = xp ? q.n_conv / kStepK : 0;
  p.ld_xp = xp ? xp->ld : 0;
  p.cand_v = fuse_argmax ? static_cast<float*>(q.workspace) : nullptr;
  p.cand_i = fuse_argmax ? reinterpret_cast<int32_t*>(static_cast<float*>(q.workspace) +
                                                      ceil_div(q.N, kTileN * pl.nw) * q.M)
                         : nullptr;
  const dim3 grid(static_cast<unsigned>(ceil_div(q.N, kTileN * (pl.nw > 0 ? pl.nw : pl.nt))),
                  static_cast<unsigned>(pl.ks));
  hipStream_t s = static_cast<hipStream_t>(stream);
  const bool norm = q.epilogue == MM_LIN_RESID_NORM;
  const bool fused_norm = norm && fused_norm_ok(p, q.dtype, q.resid, q.norm_w, q.norm_out);
  const int32_t epi = norm ? MM_LIN_RESID : q.epilogue;  // RESID_NORM = RESID + norm pass
  const int32_t main_epi = pl.ks > 1 ? kPartial : epi;
  if (xp) {
    if (q.dtype == MM_F16) launch_main_xp<MM_F16>(p, pl, grid, s);
    else launch_main_xp<MM_BF16>(p, pl, grid, s);
    return check_launch("decode_in_proj_xproj");
  }
  if (fuse_argmax) {
    if (q.dtype == MM_F16) launch_share<MM_F16>(p, kStoreArgmax, pl, grid, s);
    else launch_share<MM_BF16>(p, kStoreArgmax, pl, grid, s);
    const EmbedArgs none{nullptr, 0, nullptr, 0, 0};
    hipLaunchKernelGGL(head_argmax_kernel, dim3(static_cast<unsigned>(q.M)), dim3(256), 0, s,
                       p.cand_v, p.cand_i, static_cast<int64_t>(grid.x), q.M, argmax_ids,
                       embed ? *embed : none);
    return check_launch("decode_head_argmax");
  }
  if (use_gemv(q.M, q.N)) {
    if (q.dtype == MM_F16) launch_gemv<MM_F16>(p, epi, s);
    else launch_gemv<MM_BF16>(p, epi, s);
  } else if (pl.nw > 0) {
    if (q.dtype == MM_F16) {
      launch_share<MM_F16>(p, main_epi, pl, grid, s);
      if (fused_norm) launch_reduce_norm<MM_F16>(p, s);
      else if (pl.ks > 1) launch_reduce<MM_F16>(p, epi, s);
    } else {
      launch_share<MM_BF16>(p, main_epi, pl, grid, s);
      if (fused_norm) launch_reduce_norm<MM_BF16>(p, s);
      else if (pl.ks > 1) launch_reduce<MM_BF16>(p, epi, s);
    }
  } else if (q.dtype == MM_F16) {
    launch_main<MM_F16>(p, main_epi, pl, grid, s);
    if (fused_norm) launch_reduce_norm<MM_F16>(p, s);
    else if (pl.ks > 1) launch_reduce<MM_F16>(p, epi, s);
  } else {
    launch_main<MM_BF16>(p, main_epi, pl, grid, s);
    if (fused_norm) launch_reduce_norm<MM_BF16>(p, s);
    else if (pl.ks > 1) launch_reduce<MM_BF16>(p, epi, s);
  }
  if (norm && !fused_norm) {
    const int st = check_launch("decode_linear");
    if (st != MM_OK) return st;
    return mm_add_rmsnorm(q.resid, nullptr, q.norm_w, q.norm_out, q.M, q.N, q.ldr, 0, q.ldn, q.eps,
                          q.dtype, q.dtype, stream);
  }
  return check_launch("decode_linear");
}

}  // namespace gemm
}  // namespace mm

extern "C" {

int mm_decode_linear(const mm_linear_params* prm, void* stream) {
  mm::clear_error();
  return mm::gemm::decode_linear_core(prm, stream, nullptr);
}

size_t mm_decode_head_argmax_workspace_size(int64_t M, int64_t N, int64_t K) {
  using namespace mm::gemm;
  const size_t lin = mm_decode_linear_workspace_size(M, N, K);
  return head_fusable(M, N, K) ? std::max(lin, head_cand_bytes(M, N, K)) : lin;
}

}  // extern "C"

namespace mm {
namespace gemm {

// mm_decode_head_argmax[_embed] (embed may be NULL).
static int head_argmax(const mm_linear_params* prm, int64_t* ids, const EmbedArgs* embed,
                       void* stream) {
  if (!prm) return fail(MM_ERR_NULL_POINTER, "params is NULL");
  if (!ids) return fail(MM_ERR_NULL_POINTER, "ids is required");
  if (prm->epilogue != MM_LIN_STORE) return fail(MM_ERR_SHAPE, "the head takes the MM_LIN_STORE epilogue");
  if (prm->N > 0x3fffffffLL) return fail(MM_ERR_SHAPE, "N too large for 32-bit column indices");
  if (prm->ldy < prm->N) return fail(MM_ERR_LAYOUT, "ldy < N");
  if (!aligned(ids, 8)) return fail(MM_ERR_LAYOUT, "ids must be 8-byte aligned");
  if (!prm->x_norm_w && head_fusable(prm->M, prm->N, prm->K))
    return decode_linear_core(prm, stream, nullptr, ids, embed);
  int st = decode_linear_core(prm, stream, nullptr);
  if (st != MM_OK || prm->M == 0 || prm->N == 0) return st;
  st = mm_argmax_rows(prm->y, prm->M, prm->N, prm->ldy, prm->dtype, ids, stream);
  if (st != MM_OK || embed == nullptr) return st;
  hipLaunchKernelGGL(embed_rows_kernel, dim3(static_cast<unsigned>(prm->M)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), ids, *embed);
  return check_launch("decode_head_argmax_embed");
}

}  // namespace gemm
}  // namespace mm

extern "C" {

int mm_decode_head_argmax(const mm_linear_params* prm, int64_t* ids, void* stream) {
  mm::clear_error();
  return mm::gemm::head_argmax(prm, ids, nullptr, stream);
}

int mm_decode_head_argmax_embed(const mm_linear_params* prm, int64_t* ids, const void* table,
                                int64_t ld_table, void* rows, int64_t ld_rows, void* stream) {
  using namespace mm;
  using namespace mm::gemm;
  clear_error();
  if (!prm) return fail(MM_ERR_NULL_POINTER, "params is NULL");
  if (!table || !rows) return fail(MM_ERR_NULL_POINTER, "table and rows are required");
  if (ld_table < prm->K || ld_rows < prm->K || ld_table % 8 != 0 || ld_rows % 8 != 0 ||
      prm->K % 8 != 0 || !aligned(table, 16) || !aligned(rows, 16))
    return fail(MM_ERR_LAYOUT, "table and rows: row strides >= K (=%lld), multiples of 8, "
                "16-byte aligned", (long long)prm->K);
  const EmbedArgs e{static_cast<const u32x4*>(table), ld_table, static_cast<u32x4*>(rows),
                    ld_rows, prm->K};
  return head_argmax(prm, ids, &e, stream);
}

size_t mm_decode_in_proj_xproj_workspace_size(int64_t M, int64_t N, int64_t K, int64_t n_conv,
                                              int64_t xp_n) {
  using namespace mm::gemm;
  if (M <= 0 || N <= 0 || K <= 0 || n_conv <= 0 || xp_n <= 0) return 0;
  // enough for either path: an input RMSNorm (not known here) turns the fusion off
  const size_t two = std::max(mm_decode_linear_workspace_size(M, N, K),
                              mm_decode_linear_workspace_size(M, xp_n, n_conv));
  if (xp_fusable(M, N, K, n_conv, xp_n, false))
    return std::max(xp_workspace(M, N, K, n_conv, xp_n), two);
  return two;
}

int mm_decode_in_proj_xproj(const mm_linear_params* prm, const void* xp_w_packed, int64_t xp_n,
                            void* xp_y, int64_t ld_xp, void* stream) {
  using namespace mm;
  using namespace mm::gemm;
  clear_error();
  if (!prm) return fail(MM_ERR_NULL_POINTER, "params is NULL");
  if (prm->epilogue != MM_LIN_CONV) return fail(MM_ERR_SHAPE, "in_proj needs the MM_LIN_CONV epilogue");
  if (!xp_w_packed || !xp_y) return fail(MM_ERR_NULL_POINTER, "xp_w_packed and xp_y are required");
  if (xp_n < 1 || xp_n > 0x7fffffffLL) return fail(MM_ERR_SHAPE, "xp_n=%lld out of range", (long long)xp_n);
  if (ld_xp < xp_n) return fail(MM_ERR_LAYOUT, "ld_xp < xp_n");
  if (!aligned(xp_w_packed, 16)) return fail(MM_ERR_LAYOUT, "xp_w_packed must be 16-byte aligned");
  if (prm->n_conv % kChunkK != 0 || prm->ldc % 8 != 0 || !aligned(prm->conv_out, 16))
    return fail(MM_ERR_LAYOUT, "x_proj's K (n_conv) must be a multiple of %d and conv_out rows "
                "16-byte aligned", kChunkK);
  const mm_linear_params& q = *prm;
  if (xp_fusable(q.M, q.N, q.K, q.n_conv, xp_n, q.x_norm_w != nullptr)) {
    const XpArgs xa{xp_w_packed, xp_n, xp_y, ld_xp};
    return decode_linear_core(prm, stream, &xa);
  }
  int st = decode_linear_core(prm, stream, nullptr);
  if (st != MM_OK) return st;
  mm_linear_params x = {};
  x.x = q.conv_out;
  x.w_packed = xp_w_packed;
  x.y = xp_y;
  x.M = q.M;
  x.N = xp_n;
  x.K = q.n_conv;
  x.ldx = q.ldc;
  x.ldy = ld_xp;
  x.dtype = q.dtype;
  x.epilogue = MM_LIN_STORE;
  x.workspace = q.workspace;
  x.workspace_bytes = q.workspace_bytes;
  return decode_linear_core(&x, stream, nullptr);
}

}  // extern "C"
