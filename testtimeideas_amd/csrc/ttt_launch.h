// ttt_launch.h — host-side launchers of the gfx950 attention kernels (one per
// kernel family), called by the C ABI in ttt_capi.hip after validation.
#pragma once

#include <hip/hip_runtime.h>

#include "ttt_common.h"

namespace ttt {

// dtype codes match ttt_dtype in include/ttt_attn.h.
enum : int { kF16 = 0, kBF16 = 1, kF32 = 2 };

// Runs `stmt` with ElemT / kD bound to the element type and head dim.
#define DISPATCH_DTYPE_D(dtype, D, ...)                                   \
  do {                                                                     \
    if ((dtype) == ::ttt::kF16) {                                          \
      typedef _Float16 ElemT;                                              \
      if ((D) == 64) { constexpr int kD = 64; __VA_ARGS__; }                      \
      if ((D) == 128) { constexpr int kD = 128; __VA_ARGS__; }                    \
    } else if ((dtype) == ::ttt::kBF16) {                                  \
      typedef __bf16 ElemT;                                                \
      if ((D) == 64) { constexpr int kD = 64; __VA_ARGS__; }                      \
      if ((D) == 128) { constexpr int kD = 128; __VA_ARGS__; }                    \
    } else if ((dtype) == ::ttt::kF32) {                                   \
      typedef float ElemT;                                                 \
      if ((D) == 64) { constexpr int kD = 64; __VA_ARGS__; }                      \
      if ((D) == 128) { constexpr int kD = 128; __VA_ARGS__; }                    \
    }                                                                      \
  } while (0)

// Which outputs a sum-combine finishes (see ttt_combine.hip).
enum : int { kOutO = 0, kOutDQ = 1, kOutDKDV = 2, kOutDV = 3, kOutGKGV = 4 };

// Partial accumulators and row scalars per chunk, by kernel family.
// kFamFwdPairs: the O + LSE forward over pairs of row blocks (k_fwd_lse).
enum : int { kFamFwdOnline = 0, kFamFwdP = 1, kFamDq = 2, kFamDkdv = 3, kFamGgRow = 4, kFamGgRowGdo = 5,
             kFamGgCol = 6, kFamFwdPairs = 7, kNumFams = 8 };
constexpr int kFamNacc[] = {1, 1, 1, 2, 3, 5, 2, 1};
constexpr int kFamNsc[] = {2, 2, 0, 0, 3, 3, 0, 2};

// Workgroups of a kernel (of `threads` threads) that one CU holds at once
// (HIP occupancy calculator on the current device); 0 when it cannot be
// queried.
template <typename K>
inline int occupancy_of(K kernel, int threads = kThreads) {
  int n = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, reinterpret_cast<const void*>(kernel), threads, 0) !=
      hipSuccess) {
    (void)hipGetLastError();
    return 0;
  }
  return n;
}

// Per-kernel timing (diagnostics, ttt_kernel_timing in include/ttt_attn.h):
// while enabled, each launch of a main kernel is bracketed by two HIP events
// recorded on its stream, tagged with its kind.  timing_mark does nothing
// while disabled.  TimedLaunch records the start when constructed and the end
// when it goes out of scope, around the launch statement.
enum : int { kTagFwdOnline = 0, kTagFwdStats = 1, kTagFwdP = 2, kTagDq = 3, kTagDkdv = 4, kTagGgRow = 5,
             kTagGgCol = 6, kNumTags = 7 };
void timing_mark(hipStream_t st, int tag, bool end);
struct TimedLaunch {
  hipStream_t st;
  int tag;
  TimedLaunch(hipStream_t s, int t) : st(s), tag(t) { timing_mark(st, tag, false); }
  ~TimedLaunch() { timing_mark(st, tag, true); }
};

// The problem has a key window or an additive bias: launches run the kernels'
// XM instantiation.
inline bool extended_mask(const Params& a) { return a.win > 0 || a.bias.p != nullptr; }

// The O + LSE forward can run k_fwd_lse, whose workgroups take pairs of row
// blocks (128 rows; split causal walks in chunks of an even number of
// tiles), for 16-bit problems without a window or bias; k_fwd_online takes
// 64-row blocks.  block_rows: the problem's choice (0 = the library's: row
// pairs at D = 64, where they measured faster, and 64-row blocks at
// D = 128, where the pair kernel runs one wave per SIMD and measured
// slower: b4 h16 T8192 d128 bf16 causal 1.46 against 1.36 ms).
inline bool fwd_pairs_allowed(int dtype, bool xm) { return dtype != kF32 && !xm; }
inline bool fwd_row_pairs(int dtype, int D, bool xm, int block_rows) {
  return fwd_pairs_allowed(dtype, xm) && (block_rows == 128 || (block_rows == 0 && D == 64));
}

// Occupancy of the kernels a launch of each family runs (the smaller one when
// it runs two); xm selects the window/bias instantiation.
int occupancy_fwd(int dtype, int D, bool write_p, bool xm);
int occupancy_fwd_pairs(int dtype, int D);
int occupancy_dq(int dtype, int D, bool load_p, bool xm);
int occupancy_dkdv(int dtype, int D, bool load_p, bool xm);
// Grad-grad entry points: ttt_gg.hip is built into one object per head dim
// (and, at D = 128, per 16-bit / 16-bit with GdO / fp32), suffixed 64, 128h,
// 128hg and 128f.
#define TTT_GG_CAT2(a, b) a##b
#define TTT_GG_CAT(a, b) TTT_GG_CAT2(a, b)
#define TTT_GG_NAME(name) TTT_GG_CAT(name, TTT_GG_SUFFIX)
int occupancy_gg_row64(int dtype, bool load_p, bool gdo, bool xm);
int occupancy_gg_row128h(int dtype, bool load_p, bool gdo, bool xm);
int occupancy_gg_row128hg(int dtype, bool load_p, bool gdo, bool xm);
int occupancy_gg_row128f(int dtype, bool load_p, bool gdo, bool xm);
int occupancy_gg_col64(int dtype, bool load_p, bool xm);
int occupancy_gg_col128h(int dtype, bool load_p, bool xm);
int occupancy_gg_col128f(int dtype, bool load_p, bool xm);
inline int occupancy_gg_row(int dtype, int D, bool load_p, bool gdo, bool xm) {
  if (D == 64) return occupancy_gg_row64(dtype, load_p, gdo, xm);
  if (D == 128)
    return dtype == kF32 ? occupancy_gg_row128f(dtype, load_p, gdo, xm)
           : gdo         ? occupancy_gg_row128hg(dtype, load_p, gdo, xm)
                         : occupancy_gg_row128h(dtype, load_p, gdo, xm);
  return 0;
}
inline int occupancy_gg_col(int dtype, int D, bool load_p, bool xm) {
  if (D == 64) return occupancy_gg_col64(dtype, load_p, xm);
  if (D == 128) return dtype == kF32 ? occupancy_gg_col128f(dtype, load_p, xm) : occupancy_gg_col128h(dtype, load_p, xm);
  return 0;
}

hipError_t launch_fwd(int dtype, int D, const Params& a, bool write_p, hipStream_t st);
// Zeros into the tiles of P that the forward's P pass does not write.
hipError_t launch_fill_masked_p(int dtype, const Params& a, hipStream_t st);
hipError_t launch_combine_sum(int dtype, int D, const Params& a, int which, hipStream_t st);
hipError_t launch_combine_fwd(int dtype, int D, const Params& a, hipStream_t st);
hipError_t launch_combine_gg_row(int dtype, int D, const Params& a, bool gdo, hipStream_t st);
// combine = false leaves a split dQ's partials for the dK/dV launch that
// follows (launch_bwd_dkdv with dq_combine = that launch's parameters), which
// finishes them in workgroups appended to its grid.
hipError_t launch_bwd_dq(int dtype, int D, const Params& a, bool load_p, hipStream_t st, bool combine = true);
hipError_t launch_bwd_dkdv(int dtype, int D, const Params& a, bool load_p, bool dv_only, hipStream_t st,
                           const Params* dq_combine = nullptr);
hipError_t launch_bwd_rowsum(int dtype, int D, const Params& a, hipStream_t st);
// The grad-grad row launch with combine = false finishes only E and F of its
// split blocks (launch_combine_gg_ef); the column launch that follows, given
// rowc = the row launch's parameters, sums GQ (and GdO) in workgroups
// appended to its grid.
hipError_t launch_combine_gg_ef(const Params& a, hipStream_t st);
hipError_t launch_gg_row64(int dtype, const Params& a, bool load_p, bool want_gdout, hipStream_t st, bool combine);
hipError_t launch_gg_row128h(int dtype, const Params& a, bool load_p, bool want_gdout, hipStream_t st, bool combine);
hipError_t launch_gg_row128hg(int dtype, const Params& a, bool load_p, bool want_gdout, hipStream_t st,
                              bool combine);
hipError_t launch_gg_row128f(int dtype, const Params& a, bool load_p, bool want_gdout, hipStream_t st, bool combine);
hipError_t launch_gg_col64(int dtype, const Params& a, bool load_p, hipStream_t st, const Params* rowc);
hipError_t launch_gg_col128h(int dtype, const Params& a, bool load_p, hipStream_t st, const Params* rowc);
hipError_t launch_gg_col128f(int dtype, const Params& a, bool load_p, hipStream_t st, const Params* rowc);
inline hipError_t launch_gg_row(int dtype, int D, const Params& a, bool load_p, bool want_gdout, hipStream_t st,
                                bool combine = true) {
  if (D == 64) return launch_gg_row64(dtype, a, load_p, want_gdout, st, combine);
  if (D == 128)
    return dtype == kF32 ? launch_gg_row128f(dtype, a, load_p, want_gdout, st, combine)
           : want_gdout  ? launch_gg_row128hg(dtype, a, load_p, want_gdout, st, combine)
                         : launch_gg_row128h(dtype, a, load_p, want_gdout, st, combine);
  return hipErrorInvalidValue;
}
inline hipError_t launch_gg_col(int dtype, int D, const Params& a, bool load_p, hipStream_t st,
                                const Params* rowc = nullptr) {
  if (D == 64) return launch_gg_col64(dtype, a, load_p, st, rowc);
  if (D == 128)
    return dtype == kF32 ? launch_gg_col128f(dtype, a, load_p, st, rowc) : launch_gg_col128h(dtype, a, load_p, st, rowc);
  return hipErrorInvalidValue;
}

}  // namespace ttt
