// Chunked selective scan for gfx950 (MI355X): mm_selective_scan_fwd[_strided].
//
// Semantics follow mamba_metal/kernels/selective_scan_chunked.metal:28-155
// (softplus cutoff :60-65, discretisation :78-79, y accumulation :126-128,
// SiLU(z) gate :140-144, final state :151-155) and the op wrapper
// mamba_metal/selective_scan.py:23-80.  The decomposition is this library's own.
//
// Work decomposition
//   * A workgroup owns a block of channels of one batch row.  dstate <= 16: 32 channels
//     and 4 waves; lane l takes channel l % 32 and the two half-waves of wave g take
//     state groups g and g + 4 of SPL = 2 states (8 groups cover 16 states); for some
//     chain counts 48 channels and 6 waves, or 16 channels and 4 waves whose quarter-waves
//     take one state each (see use_48, prefer_single_state).  dstate > 16: 64 channels
//     (one per lane) and 4 waves of SPL = 8 or 16 states.  Each lane
//     walks time SEQUENTIALLY with its SPL states in fp32 registers: the recurrence
//     costs one exp2 and four VALU ops per (channel, state, step), with no parallel-scan
//     overhead.
//   * Time is cut into segments.  Work units = (channel block, segment), numbered
//     segment-major.  A persistent grid (two or three workgroups per CU for 32-channel
//     blocks) claims units from an atomic ticket counter; a unit waits for its
//     predecessor segment's flag, reads the carried fp32 state, scans its segment,
//     writes the state and raises its own flag.  Every predecessor was claimed earlier
//     by a resident workgroup, so the wait always ends; the spin is bounded anyway.
//     Segment-major units balance any number of chains over the CUs.  With few chains
//     the split mode (see Mode) replaces the hand-off by segment summaries; its units
//     never wait, so its workgroups take them by a static stride (unit = workgroup +
//     k * grid) instead of the ticket atomic, which all workgroups of a short launch
//     would contend for at once.
//   * Per 32-step tile the workgroup runs a prologue over its (channel, time) elements
//     -- coalesced vector loads of u, delta, z along whichever axis is contiguous,
//     softplus, delta*u, D*u, SiLU(z) -- and stages delta', delta'*u and the tile's B/C
//     (packed fp32 by a small kernel) in LDS; the waves scan with LDS reads
//     software-pipelined one 4-step group ahead; the epilogue sums the state groups'
//     partial y's, adds D*u, gates and stores with vector stores.  The next tiles'
//     global loads are issued before the scan so HBM latency hides under VALU work.
//   * Exponentials run in the log2 domain: delta2 = delta' * log2(e) so exp(delta'*A)
//     = exp2(delta2 * A); the packed B carries the matching factor ln(2).
#include <algorithm>

#include "mm_common.h"

namespace mm {
namespace scan {

// Channels per workgroup: 64 (lane = channel) or, for the chained scan at dstate <= 16,
// 32 (each half-wave takes the 32 channels with its own states), 48 (6 waves) or 16
// (each quarter-wave takes the 16 channels with its own state).  kCpwMin sizes what
// depends on the count of channel blocks (flags, tickets), kCpwMax what depends on the
// padded channel count.
constexpr int kCpwMax = 64;
constexpr int kCpwMin = 16;
// dstate <= 16: 8 state groups of 2 states (dstate <= 8: of 1 state); the 16-channel
// block runs 16 groups of 1 state (see prefer_single_state).
constexpr int kGroups16 = 8;
constexpr int kSpl16 = 2;

constexpr int kT = 32;  // timesteps per tile
constexpr int kTP = kT + 4;  // padded LDS row length (floats)
// The sequence is padded to whole groups of four tiles (the tile loop is unrolled by
// four, without guards); padded steps are identity steps (delta' = 0, B = C = 0).
constexpr int kTGroup = 4;

inline int64_t padded_len(int64_t seqlen) {
  return round_up(seqlen > 1 ? seqlen : 1, kTGroup * kT);
}
// Default bound of a segment's wait for its predecessor's carried state (a wait that
// always ends, see the file comment; the bound only keeps every wave's exit finite).
constexpr int64_t kDefaultHandoffTimeoutUs = 2000000;

enum Layout { kTimeContig = 0, kChanContig = 1 };

struct Params {
  const float* A;
  const float* D;
  int64_t dim, dstate, seqlen, Lp;
  int64_t nblk_d;     // channel blocks per batch row
  int64_t ncb;        // channel blocks in total (batch * nblk_d)
  int64_t seg_tiles;  // tiles per segment
  int64_t nseg;       // segments per chain
  int64_t nunits;     // ncb * nseg
  int64_t us0, us1, us2, ds0, ds1, ds2, zs0, zs1, zs2, ys0, ys1, ys2;
  int64_t As0, As1, Ds;
  float softplus_cut;  // 20 with delta_softplus, NaN without (see delta_log2)
  int32_t vec_ok;
  int* status;  // optional persistent status word (MM_SCAN_STATUS_* bits are ORed in)
  uint64_t spin_ticks;  // hand-off wait bound in wall-clock (s_memrealtime) ticks
};

// Scan modes.  kChained: a unit starts from its predecessor's carried state (waits for
// its flag).  kSplit runs two launches over the same units: kSummary scans every segment
// from a zero state, all at once, and records the segment's local end state and its
// sum of delta2 per channel; kFromSummary then starts segment s from the state folded
// out of the summaries of segments 0 .. s-1 (h = exp2(A * sum delta2) * h + h_local),
// so no unit waits.  The split costs a second pass over the inputs; it pays when the
// chains (channel blocks) are far fewer than the workgroups the chip holds.
enum Mode { kChained = 0, kSummary = 1, kFromSummary = 2 };
// Split mode for up to this many 64-channel blocks (see split_capable); summaries of 32-
// channel blocks take the same bytes as those of half as many 64-channel blocks.
constexpr int64_t kSplitMaxChains = 128;
// Segment summaries the workspace holds (per 64-channel block and segment): 4096 in all --
// 32 segments for each of 128 blocks, 16 for 256, and up to 256 segments per block when
// there are fewer blocks (a lone chain, the reference's B=1 D=16 benchmark, then splits
// finely enough that both passes are short).
constexpr int64_t kSplitSummaries = 128 * 32;
inline int64_t split_max_seg(int64_t ncb64) {
  return std::min<int64_t>(256, kSplitSummaries / std::max<int64_t>(ncb64, 1));
}

// Workspace: [ctl: ticket counters + error word][flags: one int per 32-channel block]
// [carry: batch * dim padded to 64 * G*SPL floats][bc: packed B/C][summaries:
// ncb*split_max_seg(ncb)*(G*SPL*64 + 64) floats for ncb 64-channel blocks, only for
// dstate <= 16 and at most kSplitMaxChains blocks].  G is the number of state groups (8 for dstate
// <= 16, else 4); a 32-channel block uses half as many carry floats as a 64-channel one,
// so the layout serves either channel block.
struct WsLayout {
  size_t flags, carry, bc, sum, total;
};

// The split pays for at most kSplitMaxChains 64-channel blocks, and up to twice that for
// long sequences (>= kSplitLongTiles tiles), where a chain's walk dominates: measured at
// B=2 D=5120 (160 blocks) L=32768 2.34 -> 2.20 ms, but at L=8192 (B=8 D=1536, 192 blocks)
// 0.65 -> 0.79 ms and at L=4096 (B=3 D=5120, 240 blocks) 0.36 -> 0.43 ms, where the second
// pass over the inputs costs more than the chain walk it shortens.
constexpr int64_t kSplitLongTiles = 512;
inline bool split_capable(int64_t ncb, int64_t groups, int64_t seqlen) {
  if (groups != 8) return false;
  return ncb <= kSplitMaxChains ||
         (ncb <= 2 * kSplitMaxChains && padded_len(seqlen) / kT >= kSplitLongTiles);
}

inline int64_t max_blocks(int64_t batch, int64_t dim) { return batch * ceil_div(dim, kCpwMin); }

inline WsLayout ws_layout(int64_t batch, int64_t dim, int64_t groups, int64_t spl, int64_t seqlen) {
  const int64_t ncb = batch * ceil_div(dim, kCpwMax);
  WsLayout w;
  w.flags = 256;
  w.carry = static_cast<size_t>(round_up(w.flags + 4 * max_blocks(batch, dim), 256));
  w.bc = static_cast<size_t>(round_up(w.carry + 4 * ncb * groups * spl * kCpwMax, 256));
  w.sum = static_cast<size_t>(
      round_up(w.bc + static_cast<size_t>(4 * batch * groups * padded_len(seqlen) * 2 * spl), 256));
  w.total = w.sum;
  if (split_capable(ncb, groups, seqlen))
    w.total += static_cast<size_t>(4 * ncb * split_max_seg(ncb) * (groups * spl * kCpwMax + kCpwMax));
  return w;
}

inline void pick_shape(int64_t dstate, int* groups, int* spl) {
  // 8 waves x 2 states for dstate <= 16 (enough waves per CU to hide the exp and LDS
  // latency at one workgroup per CU); 4 waves x SPL above.
  if (dstate <= 16) {
    *groups = kGroups16;
    *spl = dstate <= 8 ? kSpl16 / 2 : kSpl16;
  } else {
    *groups = 4;
    *spl = dstate <= 32 ? 8 : 16;
  }
}

// Between one and two 32-channel chains per CU half the CUs would run two chains, which
// then set the critical path.  48-channel blocks of 6 waves make it one chain per CU where
// that many fit; their carries fit the workspace's 64-channel layout when dim rounds up
// no further for 48 than for 64.  Time-contiguous inputs in this range take the 16-channel
// blocks instead (prefer_single_state is checked first), so these serve channel-contiguous
// ones.
inline bool use_48(int64_t batch, int64_t dim, int64_t cus) {
  return batch * ceil_div(dim, 32) > cus && batch * ceil_div(dim, 48) <= cus &&
         round_up(dim, 48) <= round_up(dim, 64);
}

// Time-contiguous dstate 9..16 scans with 2-4 (not exactly 4) chains per CU in 16-channel
// blocks that the split scan does not take run 16-channel blocks with one state per lane:
// three or four resident workgroups of 4 waves per CU then hold three or four chains per
// CU, where 32-channel blocks leave some CUs one chain fewer and 48-channel blocks put 2,
// 2, 1, 1 waves on the SIMDs.  (At exactly 4 per CU the 32-channel blocks are even, 2 per
// CU, and faster: B=4 D=4096 L=8192 0.64 vs 0.69 ms; from 3 to 4 per CU the 16-channel
// blocks gained 3-9%: B=7 D=2048 0.638 -> 0.60 ms, B=5 D=3072 0.649 -> 0.61, B=2 D=7680
// 0.647 -> 0.59, B=3 D=5120 0.70 -> 0.68.)  Measured against the 32-channel blocks (fp16, L=8192): B=1 D=8704
// 0.565 -> 0.500 ms, B=2 D=5120 0.59 -> 0.545, B=3 D=4096 0.588 -> 0.557; against the
// 48-channel blocks at B=8 D=1536 (config 2) 0.568 -> 0.518-0.528 and 0.61 -> 0.60 on two
// boxes (it lost, 0.64 -> 0.68, before the scan phase ran at a raised wave priority).  It
// loses where the recurrence is VALU-bound, its single state per lane giving the scheduler
// half the independent work: B=4 D=5120 L=32768 2.78 -> 3.24 ms, B=64 D=5120 L=512 0.68 ->
// 0.84, B=16 D=1536 L=4096 0.43 -> 0.52.  A lane's update costs the same five VALU
// instructions; each wave folds its four rows' partial y's in registers (see FOLD4), so
// the epilogue sums 4 partials per (channel, step) instead of 8.
inline bool prefer_single_state(int64_t batch, int64_t dim, int64_t seqlen, int64_t cus) {
  const int64_t ncb16 = batch * ceil_div(dim, 16);
  return ncb16 > 2 * cus && ncb16 < 4 * cus &&
         !split_capable(batch * ceil_div(dim, 64), kGroups16, seqlen);
}

// ---------------------------------------------------------------------------
// B/C pack: bc[((b*G + g)*Lp + t)*2*SPL + k]       = ln2 * B[b, g*SPL + k, t]
//           bc[((b*G + g)*Lp + t)*2*SPL + SPL + k] = C[b, g*SPL + k, t]
// zero for padded states and steps.  Also clears the ticket counter and flags.
template <int DT, int SPL, int G>
__global__ __launch_bounds__(256) void pack_bc_kernel(const void* __restrict__ B,
                                                      const void* __restrict__ C,
                                                      float* __restrict__ bc,
                                                      int* __restrict__ ctl, int64_t nctl,
                                                      int64_t batch, int64_t dstate,
                                                      int64_t seqlen, int64_t Lp, int64_t Bs0,
                                                      int64_t Bs1, int64_t Bs2, int64_t Cs0,
                                                      int64_t Cs1, int64_t Cs2) {
  const int64_t gid = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (int64_t i = gid; i < nctl; i += stride) ctl[i] = 0;
  const int64_t total = batch * (G * SPL) * Lp;
  for (int64_t i = gid; i < total; i += stride) {
    const int64_t t = i % Lp;
    const int64_t n = (i / Lp) % (G * SPL);
    const int64_t b = i / (Lp * G * SPL);
    const bool ok = n < dstate && t < seqlen;
    const float bv = ok ? ld<DT>(B, b * Bs0 + n * Bs1 + t * Bs2) * kLn2 : 0.0f;
    const float cv = ok ? ld<DT>(C, b * Cs0 + n * Cs1 + t * Cs2) : 0.0f;
    const int64_t g = n / SPL, k = n % SPL;
    float* o = bc + ((b * G + g) * Lp + t) * (2 * SPL);
    o[k] = bv;
    o[SPL + k] = cv;
  }
}

// float vectors of the prologue's LDS stores and the epilogue's LDS reads
template <int W>
struct FVec;
template <>
struct FVec<4> {
  typedef float type __attribute__((ext_vector_type(4)));
};
template <>
struct FVec<2> {
  typedef float type __attribute__((ext_vector_type(2)));
};

template <int DT, int N>
struct Vec;
template <int DT>
struct Vec<DT, 8> {
  using T = typename Ty<DT>::T;
  typedef T type __attribute__((ext_vector_type(8)));
};
template <int DT>
struct Vec<DT, 4> {
  using T = typename Ty<DT>::T;
  typedef T type __attribute__((ext_vector_type(4)));
};
template <int DT>
struct Vec<DT, 2> {
  using T = typename Ty<DT>::T;
  typedef T type __attribute__((ext_vector_type(2)));
};

// delta2 = delta' * log2(e), delta' = x <= cut ? softplus(x) : x.  cut is the reference's
// softplus cutoff 20 when delta_softplus is on, NaN when it is off (every comparison with
// NaN is false: delta' = x), so the flag costs no select of its own.  fp32 inputs keep
// log1p accuracy; fp16/bf16 inputs (whose own rounding is 2^-11 / 2^-8) use
// log2(1 + 2^m) directly.
template <int DT>
__device__ __forceinline__ float delta_log2(float x, float cut) {
  const float m = x * kLog2e;
  float l;
  if constexpr (DT == MM_F32) l = log1p_exp(x) * kLog2e;
  else l = log2_hw(1.0f + exp2_hw(m));
  return x <= cut ? l : m;
}

// ---------------------------------------------------------------------------
template <int DT, int LAYOUT, int SPL, int G, bool VEC, int MODE, int CPW>
__global__ __launch_bounds__(64 * G, 1) void scan_kernel(
    const Params p, const void* __restrict__ u_, const void* __restrict__ delta_,
    const void* __restrict__ z_, void* __restrict__ y_, const float* __restrict__ bc_,
    float* __restrict__ state_out_, int* __restrict__ ctl_, float* __restrict__ carry_,
    int* __restrict__ tick_, float* __restrict__ sum_) {
  using T = typename Ty<DT>::T;
  // CPW channels per workgroup and GS = 64 G / CPW state groups.  CPW = 64: lane l takes
  // channel l, wave g state group g.  CPW = 32: the two half-waves take the same
  // channels and different states (state groups g and g + G); CPW = 16 likewise with
  // four quarter-waves (state groups g, g + G, g + 2G, g + 3G).  CPW = 48 (6 waves):
  // thread t takes channel t % 48 and state group t / 48.
  static_assert(CPW == 64 || CPW == 48 || CPW == 32 || CPW == 16, "channel block");
  constexpr int NT = 64 * G;
  static_assert(NT % CPW == 0, "whole state groups per workgroup");
  constexpr int GS = NT / CPW;
  constexpr int EPT = CPW * kT / NT;  // elements per thread per tile
  static_assert(EPT == 8 || EPT == 4 || EPT == 2, "tile split");
  using VE = typename Vec<DT, EPT>::type;
  constexpr int VW = EPT >= 4 ? 4 : 2;  // floats per LDS vector access of the prologue/epilogue
  using FV = typename FVec<VW>::type;
  constexpr int TPC = kT / EPT;        // threads per channel (time-contiguous mapping)
  constexpr int BCF = GS * kT * 2 * SPL;  // floats of B/C per tile
  constexpr int BCV = BCF / 4;
  constexpr int BCPT = (BCV + NT - 1) / NT;
  constexpr int64_t SB = GS * SPL * CPW + CPW;  // floats per segment summary

  // LDS tiles of delta2, delta2*u and the G partial y's.  Time-contiguous inputs stage
  // them channel-major ([channel][time], rows of kTP floats); channel-contiguous
  // inputs time-major ([time][channel], rows of kCP floats), so that the prologue's
  // and the epilogue's float4 accesses run along the axis each thread owns and hit
  // distinct banks either way.
  constexpr int kCP = CPW + 4;
  constexpr int TILE_F = (LAYOUT == kTimeContig) ? CPW * kTP : kT * kCP;
  __shared__ __attribute__((aligned(16))) float s_dt[TILE_F];
  __shared__ __attribute__((aligned(16))) float s_du[TILE_F];
  auto at = [](int c, int t) { return (LAYOUT == kTimeContig) ? c * kTP + t : t * kCP + c; };
  // Partial y's of the GS state groups: unpadded rows, [channel][time] with each row's 4-float
  // chunks XOR-permuted by channel (time-contiguous) so that eight consecutive lanes'
  // float4 accesses of one step group land on distinct banks, or [time][channel]
  // (channel-contiguous), conflict-free as it is.  Dropping the padding of the other
  // tiles here saves 9 KB of LDS and measured ~3% faster at config 4.
  constexpr int YT = CPW * kT;
  static_assert(kT / 4 >= 8, "the chunk permutation needs eight chunks per row");
  // 16-channel blocks along time fold their four quarter-waves' partial y's in registers
  // (the quarters are the wave's four 16-lane rows): one partial per wave is stored.
  constexpr bool FOLD4 = CPW == 16 && LAYOUT == kTimeContig && MODE != kSummary;
  constexpr int YG = FOLD4 ? G : GS;
  __shared__ __attribute__((aligned(16))) float s_y[YG][YT];
  auto aty = [](int c, int t) {
    return (LAYOUT == kTimeContig) ? c * kT + ((((t >> 2) ^ (c & 7)) << 2) | (t & 3))
                                   : t * CPW + c;
  };
  // B/C of the tile, one row of kT steps x (SPL B, SPL C) per state group.  A 32-channel
  // block's half-waves read two groups G rows apart in one instruction (a 16-channel
  // block's quarter-waves four): the 4-float pad puts those rows on different banks.
  constexpr int BCR = kT * 2 * SPL + 4;
  __shared__ __attribute__((aligned(16))) float s_bc[GS][BCR];
  __shared__ int s_ticket;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int g = __builtin_amdgcn_readfirstlane(tid >> 6);
  // this thread's channel in the block and its state group (wave-uniform when CPW = 64)
  const int lch = (64 % CPW == 0) ? (lane & (CPW - 1)) : (tid % CPW);
  const int sg = (64 % CPW == 0) ? (lane / CPW) * G + g : (tid / CPW);
  const bool has_z = z_ != nullptr;

  // Element ownership for the prologue / epilogue: consecutive threads walk the
  // contiguous axis, so a wave's vector access covers whole 128-byte rows -- along
  // time (TPC threads per channel row) or along channels (CPT threads per step row).
  constexpr int CPT = CPW / EPT;
  const int vc = (LAYOUT == kTimeContig) ? (tid / TPC) : ((tid % CPT) * EPT);
  const int vt = (LAYOUT == kTimeContig) ? ((tid % TPC) * EPT) : (tid / CPT);
  auto ec = [&](int j) { return (LAYOUT == kTimeContig) ? vc : vc + j; };
  auto et = [&](int j) { return (LAYOUT == kTimeContig) ? vt + j : vt; };

  for (int64_t round = 0;; ++round) {
    // ---- claim a unit: segment-major tickets where units wait for their predecessors
    // (every predecessor is then claimed by a running workgroup first); the split
    // passes never wait, and take units by a static stride instead of a contended
    // device-scope atomic ----
    int64_t unit;
    if constexpr (MODE == kChained) {
      if (tid == 0) s_ticket = atomicAdd(tick_, 1);
      __syncthreads();
      unit = s_ticket;
      __syncthreads();
    } else {
      unit = static_cast<int64_t>(blockIdx.x) + round * gridDim.x;
    }
    if (unit >= p.nunits) break;
    const int64_t cb = unit % p.ncb;
    const int64_t seg = unit / p.ncb;
    const int64_t b = cb / p.nblk_d;
    const int64_t d0 = (cb % p.nblk_d) * CPW;
    const int64_t tile0 = seg * p.seg_tiles;
    const int64_t tile1 = std::min<int64_t>(tile0 + p.seg_tiles, p.Lp / kT);

    // ---- per-lane constants ----
    float Av[SPL], h[SPL];
    float dsum = 0.0f;  // kSummary: sum of delta2 over the segment (this lane's channel)
    {
      const int64_t d = d0 + lch;
#pragma unroll
      for (int k = 0; k < SPL; ++k) {
        const int64_t n = static_cast<int64_t>(sg) * SPL + k;
        Av[k] = (d < p.dim && n < p.dstate) ? p.A[d * p.As0 + n * p.As1] : 0.0f;
        h[k] = 0.0f;
      }
    }
    float Dv[EPT];
#pragma unroll
    for (int j = 0; j < EPT; ++j) {
      const int64_t d = d0 + ec(j);
      Dv[j] = (p.D != nullptr && d < p.dim) ? p.D[d * p.Ds] : 0.0f;
    }

    // Input tiles are loaded in pairs, two tiles ahead: the loads of tiles 2k and 2k+1
    // are issued together, in the prologue of tile 2k-2.  With 2-byte inputs along time
    // a 32-step tile is half of each channel row's 128-byte line; requesting both
    // halves back to back means no line has to survive in L2 between tiles (rows
    // 2^k bytes apart share L2 sets, and the y stores push such lines out).
    // Slots are named variables passed by reference to always-inlined lambdas, so they
    // stay in registers (an array indexed by slot would be moved to LDS).
    VE ru0, rd0, rz0, ru1, rd1, rz1, ru2, rd2, rz2, ru3, rd3, rz3;
    float4 rbc0[BCPT], rbc1[BCPT], rbc2[BCPT], rbc3[BCPT];
#define MM_SLOT(i) ru##i, rd##i, rz##i, rbc##i
    // All loads are unconditional from clamped, in-bounds addresses (elements outside
    // the tensors read element (b, 0, 0); z, when absent, reads u; steps past the padded
    // length read step 0 of B/C): the prologue masks those elements and the epilogue
    // never stores them.  Guarded loads would make the compiler wait for every
    // outstanding load at the first use, which defeats the prefetch.
    const T* const zsrc = static_cast<const T*>(has_z ? z_ : u_);
    const int64_t zs0 = has_z ? p.zs0 : p.us0, zs1 = has_z ? p.zs1 : p.us1,
                  zs2 = has_z ? p.zs2 : p.us2;
    // Per-unit bases, so that a tile only adds its step offset: the vector path has unit
    // stride along its contiguous axis (time for time-contiguous inputs); rows past dim
    // read channel 0.  B/C: this thread's float4 slots of the packed tile.
    const float* bcb[BCPT];
#pragma unroll
    for (int i = 0; i < BCPT; ++i) {
      const int v = (tid + i * NT) % BCV;
      const int gg = v / (kT * 2 * SPL / 4), rest = v % (kT * 2 * SPL / 4);
      bcb[i] = bc_ + (b * GS + gg) * p.Lp * (2 * SPL) + rest * 4;
    }
    const int64_t dcl = (d0 + vc < p.dim) ? d0 + vc : 0;
    const T* const ub = static_cast<const T*>(u_) + b * p.us0 + dcl * p.us1;
    const T* const db = static_cast<const T*>(delta_) + b * p.ds0 + dcl * p.ds1;
    const T* const zb = zsrc + b * zs0 + dcl * zs1;
    auto load_raw = [&](VE& ru, VE& rd, VE& rz, float4 (&rbc)[BCPT], int64_t t0)
                        __attribute__((always_inline)) {
      const int64_t tb = t0 < p.Lp ? t0 : 0;
#pragma unroll
      for (int i = 0; i < BCPT; ++i)
        rbc[i] = *reinterpret_cast<const float4*>(bcb[i] + tb * (2 * SPL));
      if constexpr (VEC) {
        const int64_t tc = (t0 + vt < p.seqlen) ? t0 + vt : 0;
        if constexpr (LAYOUT == kTimeContig) {  // unit stride along time
          ru = *reinterpret_cast<const VE*>(ub + tc);
          rd = *reinterpret_cast<const VE*>(db + tc);
          if constexpr (MODE != kSummary) rz = *reinterpret_cast<const VE*>(zb + tc);
        } else {
          ru = *reinterpret_cast<const VE*>(ub + tc * p.us2);
          rd = *reinterpret_cast<const VE*>(db + tc * p.ds2);
          if constexpr (MODE != kSummary) rz = *reinterpret_cast<const VE*>(zb + tc * zs2);
        }
      } else {
#pragma unroll
        for (int j = 0; j < EPT; ++j) {
          const bool in = (d0 + ec(j) < p.dim) && (t0 + et(j) < p.seqlen);
          const int64_t dc = in ? d0 + ec(j) : 0, tc = in ? t0 + et(j) : 0;
          ru[j] = static_cast<const T*>(u_)[b * p.us0 + dc * p.us1 + tc * p.us2];
          rd[j] = static_cast<const T*>(delta_)[b * p.ds0 + dc * p.ds1 + tc * p.ds2];
          if constexpr (MODE != kSummary) rz[j] = zsrc[b * zs0 + dc * zs1 + tc * zs2];
        }
      }
    };

    load_raw(MM_SLOT(0), tile0 * kT);
    load_raw(MM_SLOT(1), (tile0 + 1) * kT);

    // ---- carried state from the previous segment of this chain ----
    if (MODE == kFromSummary && seg > 0) {
      // Fold the summaries of segments 0 .. seg-1 (written by the kSummary launch), in
      // order.  Their loads are independent of the fold, so they are issued kFold
      // segments at a time (clamped to segment seg-1, whose extra copies are not
      // folded): one memory round trip per kFold segments instead of one per segment.
      constexpr int kFold = 8;
      for (int64_t j0 = 0; j0 < seg; j0 += kFold) {
        float dlv[kFold], hlv[kFold][SPL];
#pragma unroll
        for (int q = 0; q < kFold; ++q) {
          const int64_t j = j0 + q < seg ? j0 + q : seg - 1;
          const float* sb = sum_ + (cb * p.nseg + j) * SB;
          dlv[q] = sb[GS * SPL * CPW + lch];
#pragma unroll
          for (int k = 0; k < SPL; ++k) hlv[q][k] = sb[(sg * CPW + lch) * SPL + k];
        }
#pragma unroll
        for (int q = 0; q < kFold; ++q) {
          if (j0 + q >= seg) break;
#pragma unroll
          for (int k = 0; k < SPL; ++k)
            h[k] = __builtin_fmaf(exp2_decay<DT>(Av[k] * dlv[q]), h[k], hlv[q][k]);
        }
      }
    }
    if (MODE == kChained && seg > 0) {
      if (tid == 0) {
        // Bounded by wall-clock time (never expected to expire; it keeps every wave's
        // exit finite).  Once one wait of this call has given up, y is invalid anyway
        // and later waits return at once, so a failing call ends within one bound.
        const uint64_t t_start = wall_clock64();
        while (__hip_atomic_load(&ctl_[64 + cb], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) <
               static_cast<int>(seg)) {
          if (__hip_atomic_load(&ctl_[1], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0) break;
          __builtin_amdgcn_s_sleep(1);
          if (wall_clock64() - t_start > p.spin_ticks) {
            __hip_atomic_store(&ctl_[1], MM_SCAN_STATUS_HANDOFF_TIMEOUT, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
            if (p.status != nullptr)
              __hip_atomic_fetch_or(p.status, MM_SCAN_STATUS_HANDOFF_TIMEOUT, __ATOMIC_RELAXED,
                                    __HIP_MEMORY_SCOPE_AGENT);
            break;
          }
        }
      }
      __syncthreads();
      float* cp = carry_ + ((cb * GS + sg) * CPW + lch) * SPL;
#pragma unroll
      for (int k = 0; k < SPL; ++k)
        h[k] = __hip_atomic_load(cp + k, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    // Take delivery of the carried state here: the tile loop then finds no load pending
    // on h, so it carries no wait for one (that wait also covered the tiles' prefetches).
#pragma unroll
    for (int k = 0; k < SPL; ++k) asm volatile("" : "+v"(h[k]));

    // process(slot, tile, slot a, slot b, issue): scan tile from the first slot; with
    // issue, load tiles tile + 2 and tile + 3 into slots a and b (both free: consumed
    // two tiles ago).
    auto process = [&](VE& ru, VE& rd, VE& rz, float4 (&rbc)[BCPT], int64_t tile, VE& uA, VE& dA,
                       VE& zA, float4 (&bcA)[BCPT], VE& uB, VE& dB, VE& zB, float4 (&bcB)[BCPT],
                       bool issue) __attribute__((always_inline)) {
      const int64_t t0 = tile * kT;
      // Tiles wholly inside the tensors (every tile when seqlen and dim are whole tiles
      // and blocks) skip the masking below on a wave-uniform branch.
      const bool full = (t0 + kT <= p.seqlen) && (d0 + CPW <= p.dim);

      // ---- prologue ----
      // Wave priority: the scan phase issues ahead of the prologue / epilogue of the other
      // workgroups sharing the SIMD (their loads and LDS round trips wait either way),
      // which measured config 4 2.722 -> 2.646 ms and the 2.8B prefill scan 0.661 -> 0.646
      // ms (config 2 on the 48-channel blocks unchanged; on the 16-channel blocks, three
      // waves per SIMD, it turned a loss into a gain: see prefer_single_state); reversed
      // (prologue / epilogue first) it was slower (2.76 ms).
      __builtin_amdgcn_s_setprio(0);
      float yskip[EPT], gate[EPT], dtv[EPT], duv[EPT];
#pragma unroll
      for (int j = 0; j < EPT; ++j) {
        const float uu = Ty<DT>::f(ru[j]);
        const float dr = Ty<DT>::f(rd[j]);
        const float d2 = delta_log2<DT>(dr, p.softplus_cut);
        dtv[j] = d2;
        duv[j] = d2 * uu;
        if constexpr (MODE != kSummary) {
          yskip[j] = Dv[j] * uu;
          gate[j] = has_z ? silu_f(Ty<DT>::f(rz[j])) : 1.0f;
        }
      }
      if (!full) {
        // The empty volatile asm cannot be speculated, so the compiler keeps this a
        // branch instead of turning it into selects that every tile would execute.
        asm volatile("");
#pragma unroll
        for (int j = 0; j < EPT; ++j) {
          const bool in = (d0 + ec(j) < p.dim) && (t0 + et(j) < p.seqlen);
          dtv[j] = in ? dtv[j] : 0.0f;  // identity step outside the tensor
          duv[j] = in ? duv[j] : 0.0f;
        }
      }
#pragma unroll
      for (int j = 0; j < EPT; j += VW) {
        FV dv, uv;
#pragma unroll
        for (int e = 0; e < VW; ++e) {
          dv[e] = dtv[j + e];
          uv[e] = duv[j + e];
        }
        const int o = (LAYOUT == kTimeContig) ? at(vc, vt + j) : at(vc + j, vt);
        *reinterpret_cast<FV*>(&s_dt[o]) = dv;
        *reinterpret_cast<FV*>(&s_du[o]) = uv;
      }
#pragma unroll
      for (int i = 0; i < BCPT; ++i) {
        const int v = tid + i * NT;
        if (v < BCV) {
          constexpr int VPG = kT * 2 * SPL / 4;  // float4s per state group
          *reinterpret_cast<float4*>(&s_bc[v / VPG][(v % VPG) * 4]) = rbc[i];
        }
      }
      if (issue) {  // in flight during the next two tiles' scans
        load_raw(uA, dA, zA, bcA, t0 + 2 * kT);
        load_raw(uB, dB, zB, bcB, t0 + 3 * kT);
      }
      __syncthreads();

      __builtin_amdgcn_s_setprio(2);
      // ---- scan: lane = channel (mod CPW), wave and half-wave = state group; LDS reads
      // one group ahead ----
      struct Grp {
        float4 d4, u4;
        float bc[4][2 * SPL];
      };
      auto fetch = [&](int tt, Grp& gr) {
        if constexpr (LAYOUT == kTimeContig) {
          gr.d4 = *reinterpret_cast<const float4*>(&s_dt[at(lch, tt)]);
          gr.u4 = *reinterpret_cast<const float4*>(&s_du[at(lch, tt)]);
        } else {
          gr.d4 = make_float4(s_dt[at(lch, tt)], s_dt[at(lch, tt + 1)], s_dt[at(lch, tt + 2)],
                              s_dt[at(lch, tt + 3)]);
          gr.u4 = make_float4(s_du[at(lch, tt)], s_du[at(lch, tt + 1)], s_du[at(lch, tt + 2)],
                              s_du[at(lch, tt + 3)]);
        }
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
          for (int k = 0; k < 2 * SPL; ++k) gr.bc[j][k] = s_bc[sg][(tt + j) * 2 * SPL + k];
      };
      Grp cur, nxt;
      constexpr bool kPipe = SPL <= 4;
      if (kPipe) fetch(0, nxt);
      constexpr int kGroupUnroll = kPipe ? 8 : 1;
#pragma unroll kGroupUnroll
      for (int tt = 0; tt < kT; tt += 4) {
        if (kPipe) {
          cur = nxt;
          if (tt + 4 < kT) fetch(tt + 4, nxt);
          // Keep the next group's LDS reads here, ahead of this group's arithmetic: left
          // alone, the scheduler sinks them to just before their use and the wave then
          // waits out each read's latency (measured: config 4 2.886 -> 2.781 ms, config 2
          // 0.606 -> 0.577 ms, bit-identical output).
          __builtin_amdgcn_sched_barrier(0);
        } else {
          fetch(tt, cur);
        }
        const float dts[4] = {cur.d4.x, cur.d4.y, cur.d4.z, cur.d4.w};
        const float dus[4] = {cur.u4.x, cur.u4.y, cur.u4.z, cur.u4.w};
        if constexpr (MODE == kSummary) {
#pragma unroll
          for (int j = 0; j < 4; ++j) {
#pragma unroll
            for (int k = 0; k < SPL; ++k) {
              const float a = exp2_decay<DT>(dts[j] * Av[k]);
              h[k] = __builtin_fmaf(a, h[k], dus[j] * cur.bc[j][k]);
            }
            dsum += dts[j];
          }
          // Without the y stores nothing observable follows the updates, and the compiler
          // sinks the whole recurrence past the later barriers, keeping every tile's LDS
          // values live (and spilling).  An opaque use per group keeps it in order.
#pragma unroll
          for (int k = 0; k < SPL; ++k) asm volatile("" : "+v"(h[k]));
          asm volatile("" : "+v"(dsum));
          continue;
        }
        float ys[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          float acc = 0.0f;
#pragma unroll
          for (int k = 0; k < SPL; ++k) {
            const float a = exp2_decay<DT>(dts[j] * Av[k]);
            h[k] = __builtin_fmaf(a, h[k], dus[j] * cur.bc[j][k]);
            acc = __builtin_fmaf(h[k], cur.bc[j][SPL + k], acc);
          }
          ys[j] = acc;
        }
        if constexpr (FOLD4) {
          // sum over the wave's four rows (quarters, state groups g, g+G, g+2G, g+3G) of
          // steps tt..tt+3: the 32-lane swaps add rows r and r+2 (steps 0 and 2 stay in
          // the lower half, 1 and 3 in the upper), the 16-lane swap then rows r and r+1;
          // row q ends with step tt+q's sum, (q0 + q2) + (q1 + q3)
          const auto a02 = __builtin_amdgcn_permlane32_swap(__float_as_uint(ys[0]), __float_as_uint(ys[2]),
                                                            false, false);
          const auto a13 = __builtin_amdgcn_permlane32_swap(__float_as_uint(ys[1]), __float_as_uint(ys[3]),
                                                            false, false);
          const float s02 = __uint_as_float(a02[0]) + __uint_as_float(a02[1]);
          const float s13 = __uint_as_float(a13[0]) + __uint_as_float(a13[1]);
          const auto b = __builtin_amdgcn_permlane16_swap(__float_as_uint(s02), __float_as_uint(s13),
                                                          false, false);
          s_y[g][aty(lch, tt + (lane >> 4))] = __uint_as_float(b[0]) + __uint_as_float(b[1]);
        } else if constexpr (LAYOUT == kTimeContig) {
          *reinterpret_cast<float4*>(&s_y[sg][aty(lch, tt)]) = make_float4(ys[0], ys[1], ys[2], ys[3]);
        } else {
#pragma unroll
          for (int j = 0; j < 4; ++j) s_y[sg][aty(lch, tt + j)] = ys[j];
        }
      }
      __syncthreads();
      if constexpr (MODE == kSummary) return;

      // ---- epilogue: y = (sum_g partial + D*u) * SiLU(z) -> HBM ----
      __builtin_amdgcn_s_setprio(0);
      float yv[EPT];
#pragma unroll
      for (int j = 0; j < EPT; ++j) yv[j] = yskip[j];
      {
        // all G partial reads in flight before the (in-order) sum
        FV part[YG][EPT / VW];
#pragma unroll
        for (int gg = 0; gg < YG; ++gg)
#pragma unroll
          for (int j = 0; j < EPT; j += VW)
            part[gg][j / VW] = *reinterpret_cast<const FV*>(
                &s_y[gg][(LAYOUT == kTimeContig) ? aty(vc, vt + j) : aty(vc + j, vt)]);
#pragma unroll
        for (int gg = 0; gg < YG; ++gg)
#pragma unroll
          for (int j = 0; j < EPT; j += VW)
#pragma unroll
            for (int e = 0; e < VW; ++e) yv[j + e] += part[gg][j / VW][e];
      }
      VE ry;
#pragma unroll
      for (int j = 0; j < EPT; ++j) ry[j] = Ty<DT>::from(yv[j] * gate[j]);
      if constexpr (VEC) {
        T* const yp = static_cast<T*>(y_) + b * p.ys0 + (d0 + vc) * p.ys1 +
                      (LAYOUT == kTimeContig ? t0 + vt : (t0 + vt) * p.ys2);
        if (full || ((d0 + vc < p.dim) && (t0 + vt < p.seqlen))) *reinterpret_cast<VE*>(yp) = ry;
      } else {
#pragma unroll
        for (int j = 0; j < EPT; ++j) {
          const int64_t d = d0 + ec(j), t = t0 + et(j);
          if (d < p.dim && t < p.seqlen)
            static_cast<T*>(y_)[b * p.ys0 + d * p.ys1 + t * p.ys2] = ry[j];
        }
      }
    };
    // tile1 - tile0 is a multiple of kTGroup (padded length, whole-group segments)
    static_assert(kTGroup == 4, "the loop below is unrolled by four");
    for (int64_t tile = tile0; tile < tile1; tile += kTGroup) {
      process(MM_SLOT(0), tile, MM_SLOT(2), MM_SLOT(3), true);
      process(MM_SLOT(1), tile + 1, MM_SLOT(2), MM_SLOT(3), false);
      process(MM_SLOT(2), tile + 2, MM_SLOT(0), MM_SLOT(1), true);
      process(MM_SLOT(3), tile + 3, MM_SLOT(0), MM_SLOT(1), false);
    }
#undef MM_SLOT

    // ---- hand the state on, or write the final state ----
    if constexpr (MODE == kSummary) {
      float* sb = sum_ + (cb * p.nseg + seg) * SB;
#pragma unroll
      for (int k = 0; k < SPL; ++k) sb[(sg * CPW + lch) * SPL + k] = h[k];
      if (sg == 0) sb[GS * SPL * CPW + lch] = dsum;
    } else if (MODE == kChained && seg + 1 < p.nseg) {
      float* cp = carry_ + ((cb * GS + sg) * CPW + lch) * SPL;
#pragma unroll
      for (int k = 0; k < SPL; ++k)
        __hip_atomic_store(cp + k, h[k], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      // Release without an L2 writeback: the carry stores are device-coherent (sc1), so
      // waiting for them to complete (vmcnt(0)) in every wave before the barrier orders
      // them before the flag store below.  A workgroup-scope fence would not wait for
      // global stores, and an agent-scope one would write back the whole L2.
      __builtin_amdgcn_s_waitcnt(0);
      __syncthreads();
      if (tid == 0)
        __hip_atomic_store(&ctl_[64 + cb], static_cast<int>(seg + 1), __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
    } else if (state_out_ != nullptr && seg + 1 == p.nseg) {
      const int64_t d = d0 + lch;
      if (d < p.dim) {
#pragma unroll
        for (int k = 0; k < SPL; ++k) {
          const int64_t n = static_cast<int64_t>(sg) * SPL + k;
          if (n < p.dstate) state_out_[(b * p.dim + d) * p.dstate + n] = h[k];
        }
      }
    }
    __syncthreads();  // LDS reuse by the next unit
  }
}

// ---------------------------------------------------------------------------
// Workgroups per CU an instantiation can keep resident on the current device; the
// caller keeps one DeviceCache per instantiation.
template <typename K>
int resident_per_cu(DeviceCache& cache, K kernel, int threads) {
  return device_cached(
      cache,
      [&] {
        int n = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, kernel, threads, 0) != hipSuccess)
          n = 0;
        return n;
      },
      1);
}

// Segments per chain.  A chain's segments run one after another (each waits for the
// carried state of the previous one), so at most min(grid, chains) units run at once and
// the makespan is about ceil(units / that) rounds of (seg_tiles + ~1 tile of per-unit
// overhead: ticket, carry hand-off, pipeline fill).  Segments are whole groups of four
// tiles (load pairs stay on whole lines; the unrolled tile loop needs no guards) and at
// least 16 tiles where the sequence allows.  Among counts whose estimate is within 2% of
// the best, the largest wins: finer units even out workgroups that run slower.
inline void pick_segments(Params& p, int64_t grid) {
  const int64_t ntiles = p.Lp / kT;
  const int64_t par = std::max<int64_t>(1, std::min<int64_t>(grid, p.ncb));
  const int64_t max_seg = std::max<int64_t>(1, std::min<int64_t>(64, ntiles / 16));
  int64_t cost[65] = {0};
  int64_t best = INT64_MAX;
  for (int64_t n = 1; n <= max_seg; ++n) {
    const int64_t st = round_up(ceil_div(ntiles, n), kTGroup);
    const int64_t ns = ceil_div(ntiles, st);
    cost[n] = (p.ncb * ns > (1LL << 30)) ? INT64_MAX : ceil_div(p.ncb * ns, par) * (st + 1);
    best = std::min(best, cost[n]);
  }
  int64_t pick = 1;
  for (int64_t n = 1; n <= max_seg; ++n)
    if (cost[n] != INT64_MAX && cost[n] * 50 <= best * 51) pick = n;
  p.seg_tiles = round_up(ceil_div(ntiles, pick), kTGroup);
  p.nseg = ceil_div(ntiles, p.seg_tiles);
  p.nunits = p.ncb * p.nseg;
}

// Split or chained (see Mode).  In tile-times: the chained makespan is pick_segments'
// estimate; the split one is ceil(units / grid) rounds of the summary pass (~3/4 of a
// tile per tile: no epilogue, no z) plus as many of the main pass, each unit with one
// tile of overhead, plus two tiles for the second launch.  Segments of the split are
// whole groups of four tiles, at most max_seg per chain.
inline bool pick_split(Params& p, int64_t grid_sum, int64_t grid_main, int64_t max_seg) {
  const int64_t ntiles = p.Lp / kT;
  const int64_t chained4 = 4 * ceil_div(p.nunits, std::max<int64_t>(1, std::min(grid_main, p.ncb))) *
                           (p.seg_tiles + 1);
  int64_t best = INT64_MAX, best_st = 0;
  for (int64_t n = 2; n <= max_seg; ++n) {
    const int64_t st = round_up(ceil_div(ntiles, n), kTGroup);
    const int64_t ns = ceil_div(ntiles, st);
    if (ns < 2) continue;
    const int64_t units = p.ncb * ns;
    const int64_t c4 = ceil_div(units, grid_sum) * (3 * st + 4) + ceil_div(units, grid_main) * 4 * (st + 1) + 8;
    if (c4 < best) best = c4, best_st = st;
  }
  if (best_st == 0 || best >= chained4) return false;
  p.seg_tiles = best_st;
  p.nseg = ceil_div(ntiles, best_st);
  p.nunits = p.ncb * p.nseg;
  return true;
}

// Chained launch of one channel-block width: CPW channels per workgroup, G waves.
template <int DT, int LAYOUT, int SPL, int G, bool VEC, int CPW>
void launch_chained(Params p, const mm_scan_params* a, hipStream_t s, const WsLayout& w,
                    int64_t resident) {
  auto kern = scan_kernel<DT, LAYOUT, SPL, G, VEC, kChained, CPW>;
  char* ws = static_cast<char*>(a->workspace);
  int* ctl = reinterpret_cast<int*>(ws);
  float* carry = reinterpret_cast<float*>(ws + w.carry);
  const float* bc = reinterpret_cast<const float*>(ws + w.bc);
  pick_segments(p, resident);
  if (p.ncb <= resident && 3 * p.ncb > 2 * resident) {
    // Every chain has a workgroup of its own and they fill most of the grid: a chain's
    // segments could only run one after another, so one segment per chain saves the
    // hand-offs (B=2 D=5120 L=8192, 640 16-channel chains: 0.527 -> 0.479 ms; config 2
    // 0.596 -> 0.584; B=3 D=4096 0.529 -> 0.507).  With few chains the spare workgroups
    // claiming the next segments early (their first loads issued before the wait) pay
    // for the hand-offs: B=2 D=1536 L=2048, 96 chains, 0.0568 -> 0.058 ms with one segment.
    p.seg_tiles = p.Lp / kT;
    p.nseg = 1;
    p.nunits = p.ncb;
  }
  const int64_t grid = std::min<int64_t>(p.nunits, resident);
  hipLaunchKernelGGL(kern, dim3(static_cast<unsigned>(grid)), dim3(64 * G), 0, s, p, a->u,
                     a->delta, a->z, a->y, bc, a->state_out, ctl, carry, ctl, nullptr);
}

inline void set_blocks(Params& p, int64_t batch, int cpw) {
  p.nblk_d = ceil_div(p.dim, cpw);
  p.ncb = batch * p.nblk_d;
}

// GS state groups of SPL states.  dstate > 16 (GS = 4): the chained scan on 64-channel
// blocks of 4 waves.  dstate <= 16 (GS = 8): 32-channel blocks of 4 waves, split where it
// pays (few chains, see pick_split), else chained.  A 32-channel block needs half the LDS of a 64-channel one, so three
// fit a CU (three independent workgroups, one wave per SIMD each, instead of one
// workgroup with two waves per SIMD in lockstep through its barriers), and there are twice
// as many chains.  Measured against 64-channel blocks: 3.17 -> 3.05-3.11 ms at B=4 D=5120
// L=32768 (VALU busy 68% -> 73%), 0.640 -> 0.606 ms at B=8 D=1536 L=8192, with
// bit-identical results (the same per-state arithmetic, the partial sums in the same order).
template <int DT, int LAYOUT, int SPL, int GS, bool VEC>
void launch_k(Params p, const mm_scan_params* a, hipStream_t s, const WsLayout& w) {
  const int64_t cus = num_cus();
  if constexpr (GS == 8) {
    constexpr int G = GS / 2;  // waves of a 32-channel block
    set_blocks(p, a->batch, 64);
    const int64_t ncb64 = p.ncb;
    const bool split_ok = split_capable(ncb64, GS, a->seqlen) && a->workspace_bytes >= w.total;
    auto k32 = scan_kernel<DT, LAYOUT, SPL, G, VEC, kChained, 32>;
    static DeviceCache c32_cache;
    int64_t r32 = cus * resident_per_cu(c32_cache, k32, 64 * G);
    set_blocks(p, a->batch, 32);
    if (split_ok) {
      char* ws = static_cast<char*>(a->workspace);
      int* ctl = reinterpret_cast<int*>(ws);
      float* carry = reinterpret_cast<float*>(ws + w.carry);
      const float* bc = reinterpret_cast<const float*>(ws + w.bc);
      auto ksum = scan_kernel<DT, LAYOUT, SPL, G, VEC, kSummary, 32>;
      auto kmain = scan_kernel<DT, LAYOUT, SPL, G, VEC, kFromSummary, 32>;
      static DeviceCache sum_cache, main_cache;
      const int64_t rs = cus * resident_per_cu(sum_cache, ksum, 64 * G);
      const int64_t rm = cus * resident_per_cu(main_cache, kmain, 64 * G);
      pick_segments(p, r32);  // the chained estimate pick_split weighs the split against
      // 32-channel summaries take at most the bytes of the 64-channel ones
      if (pick_split(p, rs, rm, split_max_seg(ncb64))) {
        float* sum = reinterpret_cast<float*>(ws + w.sum);
        hipLaunchKernelGGL(ksum, dim3(static_cast<unsigned>(std::min(p.nunits, rs))), dim3(64 * G),
                           0, s, p, a->u, a->delta, a->z, a->y, bc, a->state_out, ctl, carry,
                           ctl, sum);
        hipLaunchKernelGGL(kmain, dim3(static_cast<unsigned>(std::min(p.nunits, rm))), dim3(64 * G),
                           0, s, p, a->u, a->delta, a->z, a->y, bc, a->state_out, ctl, carry,
                           ctl + 2, sum);
        return;
      }
    }
    // Persistent grid size, measured on 256 CUs (three workgroups fit a CU): with two to
    // three chains per CU, two workgroups per CU (B=4 D=5120 L=32768, 640 chains: 2.88 ms
    // at 512 workgroups, 3.07 at 768, 3.0-3.2 at 576); otherwise every resident slot --
    // with more chains the tickets keep three per CU evenly busy (B=8..64 x D=5120,
    // 1280-10240 chains: 1.30-1.32 ms at 768 vs 1.46-1.47 at 512; since the scan phase
    // runs at a raised wave priority also from three chains per CU: B=16 D=1536 L=4096,
    // 768 chains, 0.44 -> 0.41 ms, B=7 D=4096 L=8192 0.97 -> 0.90, B=6 D=5120 L=4096 0.535
    // -> 0.49), with fewer the chains' segment order is the critical path and spare
    // workgroups take the next segments early (B=8 D=1536 L=8192: 0.605 ms at 768, 0.627
    // at 512).
    // 48-channel blocks (see use_48), e.g. B=8 D=1536: 384 32-channel chains, 256
    // 48-channel ones on 256 CUs
    if (use_48(a->batch, a->dim, cus)) {
      auto k48 = scan_kernel<DT, LAYOUT, SPL, 6, VEC, kChained, 48>;
      static DeviceCache c48_cache;
      const int64_t r48 = cus * resident_per_cu(c48_cache, k48, 64 * 6);
      set_blocks(p, a->batch, 48);
      launch_chained<DT, LAYOUT, SPL, 6, VEC, 48>(p, a, s, w, r48);
      return;
    }
    if (p.ncb >= 2 * cus && p.ncb < 3 * cus && r32 > 2 * cus) r32 = 2 * cus;
    launch_chained<DT, LAYOUT, SPL, GS / 2, VEC, 32>(p, a, s, w, r32);
  } else if constexpr (GS == 16) {
    // 16-channel blocks of 4 waves, one state per lane (see prefer_single_state)
    auto k16 = scan_kernel<DT, LAYOUT, SPL, 4, VEC, kChained, 16>;
    static DeviceCache c16_cache;
    // three workgroups per CU up to three chains per CU, four above (the folded partial
    // y's keep a workgroup at 17.7 KB of LDS, so four fit)
    set_blocks(p, a->batch, 16);
    const int64_t r16 = cus * std::min<int64_t>(p.ncb > 3 * cus ? 4 : 3, resident_per_cu(c16_cache, k16, 256));
    launch_chained<DT, LAYOUT, SPL, 4, VEC, 16>(p, a, s, w, r16);
  } else {
    auto kern = scan_kernel<DT, LAYOUT, SPL, GS, VEC, kChained, 64>;
    static DeviceCache per_cu_cache;
    const int64_t resident = cus * resident_per_cu(per_cu_cache, kern, 64 * GS);
    set_blocks(p, a->batch, 64);
    launch_chained<DT, LAYOUT, SPL, GS, VEC, 64>(p, a, s, w, resident);
  }
}

template <int DT, int LAYOUT, int SPL, int G>
void launch(Params p, const mm_scan_params* a, hipStream_t s, const WsLayout& w) {
  if (p.vec_ok) launch_k<DT, LAYOUT, SPL, G, true>(p, a, s, w);
  else launch_k<DT, LAYOUT, SPL, G, false>(p, a, s, w);
}

// The (SPL, G) instantiation must be exactly the shape the workspace was laid out
// for (ws_layout sizes the B/C pack and the carries by groups * spl): every shape
// pick_shape can return has its own case, and anything else is an error.
inline bool shape_known(int groups, int spl) {
  return (groups == 8 && (spl == 1 || spl == 2)) || (groups == 16 && spl == 1) ||
         (groups == 4 && (spl == 2 || spl == 4 || spl == 8 || spl == 16));
}

template <int DT, int LAYOUT>
void launch_shape(Params p, const mm_scan_params* a, hipStream_t s, const WsLayout& w, int groups,
                  int spl) {
  if (groups == 8 && spl == 1) launch<DT, LAYOUT, 1, 8>(p, a, s, w);
  else if (groups == 8 && spl == 2) launch<DT, LAYOUT, 2, 8>(p, a, s, w);
  else if (groups == 16 && spl == 1) launch<DT, LAYOUT, 1, 16>(p, a, s, w);
  else if (groups == 4 && spl == 2) launch<DT, LAYOUT, 2, 4>(p, a, s, w);
  else if (groups == 4 && spl == 4) launch<DT, LAYOUT, 4, 4>(p, a, s, w);
  else if (groups == 4 && spl == 8) launch<DT, LAYOUT, 8, 4>(p, a, s, w);
  else if (groups == 4 && spl == 16) launch<DT, LAYOUT, 16, 4>(p, a, s, w);
}

template <int DT>
void launch_layout(Params p, const mm_scan_params* a, hipStream_t s, const WsLayout& w,
                   int layout, int groups, int spl) {
  if (layout == kTimeContig)
    launch_shape<DT, kTimeContig>(p, a, s, w, groups, spl);
  else
    launch_shape<DT, kChanContig>(p, a, s, w, groups, spl);
}

template <int DT>
void launch_pack(const mm_scan_params* a, int64_t Lp, int groups, int spl, const WsLayout& w,
                 int64_t nctl, hipStream_t s) {
  const int64_t total = std::max<int64_t>(a->batch * groups * spl * Lp, nctl);
  const int64_t blocks = std::min<int64_t>(ceil_div(total, 256), 65536);
  char* ws = static_cast<char*>(a->workspace);
  int* ctl = reinterpret_cast<int*>(ws);
  float* bc = reinterpret_cast<float*>(ws + w.bc);
#define MM_PACK(S, GG)                                                                          \
  hipLaunchKernelGGL((pack_bc_kernel<DT, S, GG>), dim3(static_cast<unsigned>(blocks)), dim3(256), \
                     0, s, a->B, a->C, bc, ctl, nctl, a->batch, a->dstate, a->seqlen, Lp,        \
                     a->B_stride[0], a->B_stride[1], a->B_stride[2], a->C_stride[0],             \
                     a->C_stride[1], a->C_stride[2])
  if (groups == 8 && spl == 1) MM_PACK(1, 8);
  else if (groups == 8 && spl == 2) MM_PACK(2, 8);
  else if (groups == 16 && spl == 1) MM_PACK(1, 16);
  else if (groups == 4 && spl == 2) MM_PACK(2, 4);
  else if (groups == 4 && spl == 4) MM_PACK(4, 4);
  else if (groups == 4 && spl == 8) MM_PACK(8, 4);
  else if (groups == 4 && spl == 16) MM_PACK(16, 4);
#undef MM_PACK
}

// Host-side layout analysis: which fast path the four (batch, dim, time) tensors allow.
struct Tens {
  const void* p;
  const int64_t* s;
};

void choose_layout(const mm_scan_params* a, int ept, int* layout, int* vec_ok) {
  Tens ts[4] = {{a->u, a->u_stride}, {a->delta, a->delta_stride}, {a->y, a->y_stride},
                {a->z, a->z_stride}};
  const int nt = a->z ? 4 : 3;
  bool time_c = true, chan_c = true;
  for (int i = 0; i < nt; ++i) {
    time_c = time_c && ts[i].s[2] == 1;
    chan_c = chan_c && ts[i].s[1] == 1;
  }
  *layout = time_c ? kTimeContig : chan_c ? kChanContig : kTimeContig;
  bool ok = time_c || chan_c;
  const int64_t vbytes = ept * dtype_size(a->x_dtype);
  if (ok) ok = (*layout == kTimeContig) ? a->seqlen % ept == 0 : a->dim % ept == 0;
  for (int i = 0; ok && i < nt; ++i) {
    ok = aligned(ts[i].p, vbytes);
    const int64_t other = (*layout == kTimeContig) ? ts[i].s[1] : ts[i].s[2];
    ok = ok && (other % ept == 0) && (ts[i].s[0] % ept == 0);
  }
  *vec_ok = ok ? 1 : 0;
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
  if (a->handoff_timeout_us < 0)
    return fail(MM_ERR_SHAPE, "handoff_timeout_us=%d is negative", a->handoff_timeout_us);
  const int64_t ncb = max_blocks(a->batch, a->dim);
  if (ncb > (1LL << 30)) return fail(MM_ERR_SHAPE, "too many channel blocks (%lld)", (long long)ncb);
  return MM_OK;
}

}  // namespace scan
}  // namespace mm

namespace mm {
namespace scan {

// The scan behind both entry points.  The workspace must hold the layout's total;
// with chained_min_ok (the allocation-free entry point, whose workspace is fixed) a
// workspace that holds everything but the split scan's segment summaries also runs, on
// the chained path.
int fwd(const mm_scan_params* a, void* stream, bool chained_min_ok) {
  int st = validate(a);
  if (st != MM_OK) return st;
  if (a->batch == 0 || a->dim == 0) return MM_OK;

  int groups = 8, spl = 2;
  pick_shape(a->dstate, &groups, &spl);
  if (!shape_known(groups, spl))
    return fail(MM_ERR_DSTATE, "no scan instantiation for %d groups x %d states", groups, spl);
  int layout = kTimeContig, vec_ok = 0;
  // elements per thread per tile: kT / groups for every channel block
  choose_layout(a, kT / groups, &layout, &vec_ok);
  if (groups == kGroups16 && spl == kSpl16 && layout == kTimeContig &&
      prefer_single_state(a->batch, a->dim, a->seqlen, num_cus())) {
    groups = 16;  // the same B/C and carry bytes as 8 x 2
    spl = 1;
    choose_layout(a, kT / groups, &layout, &vec_ok);
  }
  const WsLayout w = ws_layout(a->batch, a->dim, groups, spl, std::max<int64_t>(a->seqlen, 1));
  const size_t need = chained_min_ok ? w.sum : w.total;
  if (a->workspace == nullptr || a->workspace_bytes < need)
    return fail(MM_ERR_WORKSPACE, "workspace of %zu bytes required, got %zu (%s)", need,
                a->workspace_bytes, a->workspace ? "too small" : "NULL");
  if (!aligned(a->workspace, 256)) return fail(MM_ERR_WORKSPACE, "workspace must be 256-byte aligned");

  Params p;
  p.A = a->A;
  p.D = a->D;
  p.dim = a->dim;
  p.dstate = a->dstate;
  p.seqlen = a->seqlen;
  p.Lp = padded_len(a->seqlen);
  // nblk_d / ncb are set at launch, from the channel block, and seg_tiles / nseg /
  // nunits from the persistent grid size.
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
  p.softplus_cut = a->delta_softplus ? 20.0f : __builtin_nanf("");
  p.vec_ok = vec_ok;
  p.status = a->status;
  {
    // wall-clock counter rate (kHz) of this device, for the hand-off wait's time bound
    static DeviceCache rate_cache;
    const int64_t khz = device_cached(
        rate_cache,
        [] {
          int dev = 0, r = 0;
          if (hipGetDevice(&dev) != hipSuccess ||
              hipDeviceGetAttribute(&r, hipDeviceAttributeWallClockRate, dev) != hipSuccess)
            r = 0;
          return r;
        },
        100000);
    const int64_t us = a->handoff_timeout_us > 0 ? a->handoff_timeout_us : kDefaultHandoffTimeoutUs;
    p.spin_ticks = static_cast<uint64_t>(us) * static_cast<uint64_t>(khz) / 1000u;
  }

  hipStream_t s = static_cast<hipStream_t>(stream);
  const int64_t nctl = 64 + max_blocks(a->batch, a->dim);
  switch (a->bc_dtype) {
    case MM_F32: launch_pack<MM_F32>(a, p.Lp, groups, spl, w, nctl, s); break;
    case MM_F16: launch_pack<MM_F16>(a, p.Lp, groups, spl, w, nctl, s); break;
    default: launch_pack<MM_BF16>(a, p.Lp, groups, spl, w, nctl, s); break;
  }
  st = check_launch("pack_bc");
  if (st != MM_OK) return st;
  switch (a->x_dtype) {
    case MM_F32: launch_layout<MM_F32>(p, a, s, w, layout, groups, spl); break;
    case MM_F16: launch_layout<MM_F16>(p, a, s, w, layout, groups, spl); break;
    default: launch_layout<MM_BF16>(p, a, s, w, layout, groups, spl); break;
  }
  return check_launch("selective_scan");
}

// mm_scan_params of the reference-shaped (row-major contiguous) entry points.
mm_scan_params contiguous_params(const void* u, const void* delta, const float* A, const void* B,
                                 const void* C, const float* D, const void* z, void* y,
                                 float* ssm_state_out, int64_t batch, int64_t dim, int64_t dstate,
                                 int64_t seqlen, int32_t x_dtype, int32_t bc_dtype,
                                 int32_t delta_softplus) {
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
  return a;
}

}  // namespace scan
}  // namespace mm

extern "C" {

size_t mm_selective_scan_workspace_size(int64_t batch, int64_t dim, int64_t dstate,
                                        int64_t seqlen) {
  using namespace mm::scan;
  if (batch <= 0 || dim <= 0 || dstate < 1 || dstate > MM_MAX_DSTATE || seqlen < 0) return 0;
  int groups = 8, spl = 2;
  pick_shape(dstate, &groups, &spl);
  return ws_layout(batch, dim, groups, spl, std::max<int64_t>(seqlen, 1)).total;
}

int mm_selective_scan_fwd_strided(const mm_scan_params* a, void* stream) {
  mm::clear_error();
  return mm::scan::fwd(a, stream, false);
}

int mm_selective_scan_fwd(const void* u, const void* delta, const float* A, const void* B,
                          const void* C, const float* D, const void* z, void* y,
                          float* ssm_state_out, int64_t batch, int64_t dim, int64_t dstate,
                          int64_t seqlen, int32_t x_dtype, int32_t bc_dtype,
                          int32_t delta_softplus, void* workspace, size_t workspace_bytes,
                          void* stream) {
  mm_scan_params a = mm::scan::contiguous_params(u, delta, A, B, C, D, z, y, ssm_state_out, batch,
                                                 dim, dstate, seqlen, x_dtype, bc_dtype,
                                                 delta_softplus);
  a.workspace = workspace;
  a.workspace_bytes = workspace_bytes;
  return mm_selective_scan_fwd_strided(&a, stream);
}

}  // extern "C"

// ---------------------------------------------------------------------------
// Allocation-free entry point.  Its workspace is `scratch`, a file-scope device array:
// every GPU the library runs on holds its own copy (MM_SCAN_SCRATCH_BYTES) until the
// process ends.  In host code the array's name is only a stand-in for the symbol, so
// its device address is taken once per device with hipGetSymbolAddress and kept in
// scratch_ptr[device]; kernels are only ever given that address.  The launches are
// those of mm_selective_scan_fwd (the B/C pack kernel clears the work-queue counter,
// flags and status word at the start of every call, so the previous call's contents do
// not matter; the caller's optional status word receives the call's outcome).  Calls
// that overlap in time on one GPU share the array and race.
namespace {

static __device__ __align__(256) unsigned char scratch[MM_SCAN_SCRATCH_BYTES];

std::atomic<void*> scratch_ptr[mm::kMaxDevices];

// Device address of this device's `scratch` (looked up on the first call on a device).
int scratch_address(void** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess)
    return mm::fail(MM_ERR_HIP, "hipGetDevice failed: %s", hipGetErrorString(e));
  if (dev < 0 || dev >= mm::kMaxDevices)
    return mm::fail(MM_ERR_HIP, "device %d outside the library's %d-device table", dev,
                    mm::kMaxDevices);
  void* p = scratch_ptr[dev].load(std::memory_order_acquire);
  if (p == nullptr) {
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr)
      return mm::fail(MM_ERR_HIP, "hipGetSymbolAddress(scratch) failed on device %d: %s", dev,
                      hipGetErrorString(e));
    scratch_ptr[dev].store(p, std::memory_order_release);
  }
  *out = p;
  return MM_OK;
}

}  // namespace

extern "C" int mm_selective_scan_fwd_noalloc(const void* u, const void* delta, const float* A,
                                             const void* B, const void* C, const float* D,
                                             const void* z, void* y, float* ssm_state_out,
                                             int64_t batch, int64_t dim, int64_t dstate,
                                             int64_t seqlen, int32_t x_dtype, int32_t bc_dtype,
                                             int32_t delta_softplus, int32_t* status,
                                             void* stream) {
  using namespace mm;
  clear_error();
  mm_scan_params a = scan::contiguous_params(u, delta, A, B, C, D, z, y, ssm_state_out, batch, dim,
                                             dstate, seqlen, x_dtype, bc_dtype, delta_softplus);
  a.status = status;
  // host-only checks first (no HIP call before the arguments are known to be valid)
  int st = scan::validate(&a);
  if (st != MM_OK) return st;
  if (batch == 0 || dim == 0) return MM_OK;
  // The fixed array must hold at least the chained scan's share of the workspace; the
  // split scan's segment summaries are used only when they fit too.
  int groups = 8, spl = 2;
  scan::pick_shape(dstate, &groups, &spl);
  const size_t need =
      scan::ws_layout(batch, dim, groups, spl, std::max<int64_t>(seqlen, 1)).sum;
  if (need > MM_SCAN_SCRATCH_BYTES)
    return fail(MM_ERR_WORKSPACE,
                "batch=%lld dim=%lld dstate=%lld seqlen=%lld needs %zu bytes of scan workspace; "
                "the allocation-free entry point holds %zu (use mm_selective_scan_fwd with a "
                "caller-allocated workspace)",
                (long long)batch, (long long)dim, (long long)dstate, (long long)seqlen, need,
                static_cast<size_t>(MM_SCAN_SCRATCH_BYTES));
  void* ptr = nullptr;
  st = scratch_address(&ptr);
  if (st != MM_OK) return st;
  a.workspace = ptr;
  a.workspace_bytes = MM_SCAN_SCRATCH_BYTES;
  return scan::fwd(&a, stream, true);
}
