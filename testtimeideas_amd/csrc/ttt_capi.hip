// ttt_capi.hip — the extern "C" entry points declared in include/ttt_attn.h.
// Validates every argument on the host before anything is enqueued (shapes,
// null pointers, 16-byte alignment of bases and row strides, grid limits,
// workspace size), chooses the split of the streamed loop, packs the kernel
// argument block and calls the per-family launchers.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <functional>
#include <initializer_list>
#include <map>
#include <mutex>
#include <queue>
#include <tuple>
#include <vector>

#include "../../include/ttt_attn.h"
#include "ttt_launch.h"

namespace {

thread_local char g_err[512] = "";

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

// The split of a streamed loop into chunks is chosen by simulating how the
// hardware would run the launch: workgroups go to the XCDs round-robin in
// launch order and, within an XCD, to whichever of its slots frees first.
// The simulated makespan plus a small per-workgroup cost (partials, combine)
// is minimised over the chunk length.  kSlotFill is the share (percent)
// of the nominal slots (CUs x workgroups per CU from the occupancy
// calculator) the simulation assumes usable: all of them.  Causal launches
// run their shortest chunks last, so a few workgroups past the slots cost
// little (90 % against 100 %, same box: b1 h1 T16384 d64 fp16 step 2 %
// slower, b2 h4 T2048 d128 forward with P 10 % slower).  The constants were fitted to
// MI355X sweeps of every kernel family at T = 8192 and 16384, where they pick
// the measured fastest chunk length.  Without a device (workspace queries on
// a host with no GPU) the slots default to kFallbackCus x kFallbackPerCu.
constexpr int kSlotFill = 100;
constexpr int kXcds = 8;
constexpr double kWgOverheadTiles = 0.5;   // per workgroup, in tile times
constexpr double kEmptyWgTiles = 0.05;     // a workgroup whose chunk is empty
constexpr double kWgCostTiles = 0.015;     // per workgroup, added to the makespan
constexpr double kSplitTiles = 8.0;        // any split: the combine launch and the partials' traffic
                                           // (b2 h4 T2048 d128: dQ, dK/dV -6 % unsplit)
// Causal splits are considered while the blocks fill fewer than kSimBlocks
// times the slots: up to twice the slots, a causal launch's longest blocks can
// hold the makespan well above the average (b1 h4 T8192: the launch ends with
// a 128-tile block sharing its CU); beyond that, heaviest-first order
// balances it.  Measured on MI355X (b1 hH T8192 d64 fp16 causal, fwd + bwd +
// grad-grad): H = 4 -5.5 %, H = 6 -6 %, H = 8 -1 %, other H unchanged.
// Equal-length blocks (no causal mask) gain nothing from it and lose the
// combine (b2 h4 T2048 d128 grad-grad +35 % when split).
constexpr int64_t kSimBlocks = 2;
constexpr int64_t kDeferRounds = 4;        // P pass: rounds of workgroups from which stores are deferred
// P pass at d = 64: P written beyond this many bytes (half of MI355X's 256 MB
// last-level cache) is stored with the non-temporal hint.  Its readers then
// fetch it from HBM either way (b1 h1 T16384 d64 fp16 causal, 256 MB: forward
// -7 %, dQ -6 %); below it they find it in that cache (b1 h1 T8192, 64 MB:
// dQ +15 % with the hint).
constexpr int64_t kPStreamBytes = 128ll << 20;
constexpr int64_t kMaxSimWorkgroups = 16;  // x slots: larger grids are not considered
constexpr int kDkdvPerCu = 2;  // saved-P dK/dV workgroups per CU the split simulation assumes at most
constexpr int kFallbackCus = 256;
constexpr int kFallbackPerCu = 2;
// Chunks shorter than this are not worth a combine pass.
constexpr int kMinChunk = 4;
// The same for the row-pair forward, in units of two tiles: its workgroups
// spend about four tile steps on their prologue (first loads and the shifts),
// and b1 h1 T8192 d64 causal measured 25.3 us at 16-tile chunks against 28.1
// at 12 (T16384: 34-tile chunks either way).
constexpr int kMinPairChunk = 8;

size_t elem_bytes(int dtype) { return dtype == TTT_F32 ? 4 : 2; }

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Checks a [B,H,T,X] operand and copies it into a kernel View.
int take_view(const ttt_problem* pr, const ttt_view* v, const char* name, ttt::View* out) {
  if (!v || !v->data) return fail(TTT_ERR_INVALID_ARGUMENT, "%s: null pointer", name);
  if (!aligned16(v->data)) return fail(TTT_ERR_INVALID_ARGUMENT, "%s: base pointer not 16-byte aligned", name);
  const size_t eb = elem_bytes(pr->dtype);
  if ((v->stride_t * (int64_t)eb) % 16 != 0 || v->stride_t <= 0)
    return fail(TTT_ERR_INVALID_ARGUMENT, "%s: T stride %lld elements is not a positive multiple of 16 bytes",
                name, (long long)v->stride_t);
  if ((v->stride_h * (int64_t)eb) % 16 != 0 || (v->stride_b * (int64_t)eb) % 16 != 0)
    return fail(TTT_ERR_INVALID_ARGUMENT, "%s: B/H strides must be multiples of 16 bytes", name);
  out->p = v->data;
  out->sb = v->stride_b;
  out->sh = v->stride_h;
  out->st = v->stride_t;
  return TTT_OK;
}

int check_problem(const ttt_problem* pr) {
  if (!pr) return fail(TTT_ERR_INVALID_ARGUMENT, "problem: null pointer");
  if (pr->dtype != TTT_F16 && pr->dtype != TTT_BF16 && pr->dtype != TTT_F32)
    return fail(TTT_ERR_UNSUPPORTED, "dtype code %d is not f16/bf16/f32", pr->dtype);
  if (pr->head_dim != 64 && pr->head_dim != 128)
    return fail(TTT_ERR_UNSUPPORTED, "head_dim %lld: built for 64 and 128", (long long)pr->head_dim);
  if (pr->batch < 1 || pr->heads < 1 || pr->seqlen < 1)
    return fail(TTT_ERR_INVALID_ARGUMENT, "batch, heads and seqlen must be >= 1 (got %lld, %lld, %lld)",
                (long long)pr->batch, (long long)pr->heads, (long long)pr->seqlen);
  if (pr->batch * pr->heads > 65535)
    return fail(TTT_ERR_INVALID_ARGUMENT, "batch*heads = %lld exceeds 65535", (long long)(pr->batch * pr->heads));
  if (pr->seqlen > (int64_t)1 << 24)
    return fail(TTT_ERR_INVALID_ARGUMENT, "seqlen %lld exceeds 2^24", (long long)pr->seqlen);
  if (pr->causal != 0 && pr->causal != 1) return fail(TTT_ERR_INVALID_ARGUMENT, "causal must be 0 or 1");
  if (pr->split_chunk < 0) return fail(TTT_ERR_INVALID_ARGUMENT, "split_chunk must be >= 0");
  if (pr->window < 0) return fail(TTT_ERR_INVALID_ARGUMENT, "window must be >= 0");
  if (pr->window > 0 && pr->causal != 1) return fail(TTT_ERR_INVALID_ARGUMENT, "a window needs causal=1");
  if (pr->window_kind != TTT_WINDOW_SLIDING && pr->window_kind != TTT_WINDOW_LOCAL)
    return fail(TTT_ERR_INVALID_ARGUMENT, "window_kind %d is not sliding (0) or local (1)", pr->window_kind);
  if (pr->block_rows != 0 && pr->block_rows != 64 && pr->block_rows != 128)
    return fail(TTT_ERR_INVALID_ARGUMENT, "block_rows %d is not 0, 64 or 128", pr->block_rows);
  if (pr->bias.data) {
    const int64_t eb = (int64_t)elem_bytes(pr->dtype);
    if (!aligned16(pr->bias.data)) return fail(TTT_ERR_INVALID_ARGUMENT, "bias: base pointer not 16-byte aligned");
    for (const int64_t st : {pr->bias.stride_b, pr->bias.stride_h, pr->bias.stride_t})
      if (st < 0 || (st * eb) % 16 != 0)
        return fail(TTT_ERR_INVALID_ARGUMENT, "bias: strides must be >= 0 and multiples of 16 bytes");
  }
  return TTT_OK;
}

// The window the kernels apply: W >= T sees every earlier key, i.e. none.
int eff_window(const ttt_problem* pr) { return pr->window > 0 && pr->window < pr->seqlen ? pr->window : 0; }

bool has_xm(const ttt_problem* pr) { return eff_window(pr) > 0 || pr->bias.data != nullptr; }

struct Split {
  int nblk, chunk, nchunk_max;
};

// CUs of the current device (cached per device), or 0 without one.
int device_cus(int* dev_out) {
  static std::atomic<int> no_device{0};
  static std::atomic<int> cus[16];
  if (no_device.load(std::memory_order_relaxed)) return 0;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 16) {
    (void)hipGetLastError();
    no_device.store(1, std::memory_order_relaxed);
    return 0;
  }
  *dev_out = dev;
  int n = cus[dev].load(std::memory_order_relaxed);
  if (n == 0) {
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) {
      (void)hipGetLastError();
      no_device.store(1, std::memory_order_relaxed);
      return 0;
    }
    cus[dev].store(n, std::memory_order_relaxed);
  }
  return n;
}

// Workgroup slots of family `fam`'s kernel (variant load_p) on the current
// device; cached per (device, family, dtype, head dim, variant).
int64_t family_slots(const ttt_problem* pr, int fam, bool load_p) {
  static std::atomic<int> per_cu[16][ttt::kNumFams][3][2][2][2];
  int dev = 0;
  const int cus = device_cus(&dev);
  if (cus == 0) return (int64_t)kFallbackCus * kFallbackPerCu * kSlotFill / 100;
  const int dt = pr->dtype, ds = pr->head_dim == 128 ? 1 : 0, lp = load_p ? 1 : 0;
  const bool xm = has_xm(pr);
  int n = per_cu[dev][fam][dt][ds][lp][xm].load(std::memory_order_relaxed);
  if (n == 0) {
    const int D = (int)pr->head_dim;
    switch (fam) {
      case ttt::kFamFwdOnline: n = ttt::occupancy_fwd(dt, D, false, xm); break;
      case ttt::kFamFwdPairs: n = ttt::occupancy_fwd_pairs(dt, D); break;
      case ttt::kFamFwdP: n = ttt::occupancy_fwd(dt, D, true, xm); break;
      case ttt::kFamDq: n = ttt::occupancy_dq(dt, D, load_p, xm); break;
      case ttt::kFamDkdv: n = ttt::occupancy_dkdv(dt, D, load_p, xm); break;
      case ttt::kFamGgRow: n = ttt::occupancy_gg_row(dt, D, load_p, false, xm); break;
      case ttt::kFamGgRowGdo: n = ttt::occupancy_gg_row(dt, D, load_p, true, xm); break;
      default: n = ttt::occupancy_gg_col(dt, D, load_p, xm); break;
    }
    if (n <= 0) n = kFallbackPerCu;
    // The saved-P dK/dV kernels run about two workgroups per CU where the
    // occupancy calculator allows three (counters: 1.9-2.0 waves per SIMD at
    // b1 h1 T8192/16384 d64), and their splits fitted to two measured faster
    // (b1 h1 d64 fp16 causal steps, same box: T8192 -1.9 %, T16384 -0.3 %; the
    // recompute variant, +1.5 % at T8192 with the cap, keeps three, and so
    // does D = 128, where nothing was fitted).
    if (fam == ttt::kFamDkdv && load_p && D == 64 && n > kDkdvPerCu) n = kDkdvPerCu;
    per_cu[dev][fam][dt][ds][lp][xm].store(n, std::memory_order_relaxed);
  }
  return std::max<int64_t>(1, (int64_t)cus * n * kSlotFill / 100);
}

bool column_family(int fam) { return fam == ttt::kFamDkdv || fam == ttt::kFamGgCol; }

// Streamed tiles of each block of a slice in launch order: row kernels issue
// row block nblk-1-i first when causal (block i otherwise), column kernels
// column block i.  Plain causal gives nblk, nblk-1, ..., 1.
std::vector<int64_t> block_tiles(const ttt_problem* pr, bool col) {
  const int T = (int)pr->seqlen, nblk = (T + ttt::kBlk - 1) / ttt::kBlk;
  const int W = eff_window(pr), kind = pr->window_kind, causal = pr->causal;
  std::vector<int64_t> len(nblk);
  for (int i = 0; i < nblk; ++i) {
    const ttt::Range r = col ? ttt::col_block_range(i, nblk, T, causal, W, kind)
                             : ttt::row_block_range(causal ? nblk - 1 - i : i, nblk, T, causal, W, kind);
    len[i] = r.hi - r.lo;
  }
  return len;
}

// Workgroups of one (b,h) slice when every block's streamed range is cut
// into chunks of c tiles.
int64_t slice_workgroups(const std::vector<int64_t>& len, int64_t c) {
  int64_t n = 0;
  for (const int64_t l : len) n += (l + c - 1) / c;
  return n;
}

// Simulated makespan (tile times) of a launch: grid column x of slice y =
// (b,h) runs the chunk the kernels' launch_item gives it (causal_item when
// `longest_first`, else block x % nblk, chunk x / nblk); block i (launch
// order) has len[i] tiles; `slots` usable workgroup slots spread over kXcds
// XCDs.  Workgroups go to the XCDs round-robin in linear launch order; slice
// y runs on XCD y % 8 when the slices divide evenly, else each column runs
// the item xcd_local maps it to when xcd_columns holds (the kernels'
// grid_slot).  The grid is taken as nblk * k columns wide (launches that
// append combine workgroups to it are not modelled).
double simulate_launch(const std::vector<int64_t>& len, int64_t c, int64_t bh, int64_t slots, bool longest_first,
                       int64_t* nonempty) {
  const int64_t per = std::max<int64_t>(1, slots / kXcds);
  std::vector<std::priority_queue<double, std::vector<double>, std::greater<double>>> xcd(kXcds);
  for (auto& q : xcd)
    for (int64_t i = 0; i < per; ++i) q.push(0.0);
  const int64_t nblk = (int64_t)len.size();
  const int64_t lmax = *std::max_element(len.begin(), len.end());
  const int64_t k = (lmax + c - 1) / c;
  const bool by_slice = bh % kXcds == 0;
  double end = 0.0;
  int64_t idx = 0, used = 0;
  for (int64_t y = 0; y < bh; ++y)
    for (int64_t x = 0; x < nblk * k; ++x, ++idx) {
      const int xi = (by_slice || !ttt::xcd_columns((int)(nblk * k), (int)bh))
                         ? (int)x
                         : ttt::xcd_local((int)x, (int)(nblk * k));  // as grid_slot
      const ttt::Item it = (longest_first && k > 1) ? ttt::causal_item(xi, (int)nblk, (int)c)
                                                    : ttt::Item{(int)(xi % nblk), (int)(xi / nblk)};
      const int64_t t = it.blk < 0 ? 0 : std::max<int64_t>(0, std::min(c, len[it.blk] - it.ch * c));
      auto& q = xcd[by_slice ? y % kXcds : idx % kXcds];
      const double f = q.top() + (t > 0 ? (double)t + kWgOverheadTiles : kEmptyWgTiles);
      q.pop();
      q.push(f);
      end = std::max(end, f);
      used += t > 0;
    }
  *nonempty = used;
  return end;
}

// Tiles per workgroup (see above).  Chunks are at least kMinChunk tiles, and a
// split must beat no split by kSplitTiles.  Cached per shape.
// kind: 0 row blocks, 1 column blocks, 2 row-block pairs (len in their units).
// cfloor: no chunk below it is considered (0: none).
int64_t best_chunk(const ttt_problem* pr, const std::vector<int64_t>& len, int kind, int64_t bh, int64_t slots,
                   int64_t cfloor = 0) {
  static std::mutex mu;
  static std::map<std::tuple<int64_t, int, int, int, int, int64_t, int64_t, int, int64_t>, int64_t> cache;
  const auto key = std::make_tuple((int64_t)pr->seqlen, pr->causal, eff_window(pr), pr->window_kind, kind,
                                   bh, slots, pr->bias.data ? 1 : 0, cfloor);
  // plain causal launches run their chunks longest first (causal_item)
  const bool longest_first = pr->causal && !has_xm(pr);
  {
    std::lock_guard<std::mutex> lock(mu);
    const auto it = cache.find(key);
    if (it != cache.end()) return it->second;
  }
  const int64_t lmax = *std::max_element(len.begin(), len.end());
  int64_t best_c = lmax;
  double best = 0.0;
  {
    int64_t used = 0;
    best = simulate_launch(len, lmax, bh, slots, longest_first, &used) + kWgCostTiles * used;
  }
  // candidates: every length up to 64 tiles, then steps of ~3%
  const int64_t cmin = std::max<int64_t>(kind == 2 ? kMinPairChunk : kMinChunk, cfloor);
  for (int64_t c = std::min<int64_t>(cmin, lmax); c < lmax; c = c < 64 ? c + 1 : c + std::max<int64_t>(1, c / 32)) {
    if (bh * slice_workgroups(len, c) > kMaxSimWorkgroups * slots) continue;
    int64_t used = 0;
    const double cost = simulate_launch(len, c, bh, slots, longest_first, &used) + kWgCostTiles * used + kSplitTiles;
    if (cost < best) {
      best = cost;
      best_c = c;
    }
  }
  std::lock_guard<std::mutex> lock(mu);
  cache[key] = best_c;
  return best_c;
}

// The O + LSE forward over row-block pairs (kFamFwdPairs): its
// workgroups take two blocks' rows.  Causal pairs have 2(npair - i) tiles in
// launch order (the last pair of an odd block count one fewer), so the
// launch is simulated in units of two tiles, as causal_item orders it, and
// the chunk is even; other pairs have nblk tiles each.  Partials stay per
// 64-row block: nchunk_max = ceil(nblk / chunk).
bool pair_family(int fam) { return fam == ttt::kFamFwdPairs; }

Split choose_split_pairs(const ttt_problem* pr) {
  Split s;
  s.nblk = (int)((pr->seqlen + ttt::kBlk - 1) / ttt::kBlk);
  const int64_t nblk = s.nblk, npair = (nblk + 1) / 2;
  const int64_t bh = pr->batch * pr->heads;
  int64_t c;
  if (pr->split_chunk > 0) {
    c = pr->split_chunk;
  } else {
    const int64_t slots = family_slots(pr, ttt::kFamFwdPairs, false);
    const int64_t fill = (pr->causal ? kSimBlocks : 1) * slots;
    if (bh * npair >= fill) {
      c = nblk;
    } else if (pr->causal) {
      std::vector<int64_t> len(npair);
      for (int64_t i = 0; i < npair; ++i) len[i] = npair - i;
      c = 2 * best_chunk(pr, len, 2, bh, slots);
    } else {
      c = best_chunk(pr, std::vector<int64_t>(npair, nblk), 2, bh, slots);
    }
  }
  if (pr->causal && (c & 1) && c < nblk) ++c;  // causal splits: whole pairs of tiles
  s.chunk = (int)std::min<int64_t>(c, nblk);
  s.nchunk_max = (int)((nblk + s.chunk - 1) / s.chunk);
  return s;
}

Split choose_split(const ttt_problem* pr, int fam, bool load_p) {
  if (pair_family(fam)) return choose_split_pairs(pr);
  Split s;
  s.nblk = (int)((pr->seqlen + ttt::kBlk - 1) / ttt::kBlk);
  const int64_t bh = pr->batch * pr->heads;
  const bool col = column_family(fam);
  const std::vector<int64_t> len = block_tiles(pr, col);
  const int64_t lmax = *std::max_element(len.begin(), len.end());
  int64_t c;
  if (pr->split_chunk > 0) {
    c = pr->split_chunk;
  } else {
    const int64_t slots = family_slots(pr, fam, load_p);
    // Blocks of unequal length (causal or windowed) are simulated up to
    // kSimBlocks times the slots; equal blocks stop splitting at the slots.
    const int64_t fill = (pr->causal ? kSimBlocks : 1) * slots;
    // The P pass merges the statistics pass's chunks in batches of
    // kLseMergeBatch loads before its first tile: chunks past one batch cost
    // it another round trip (b1 h1 T8192 d64 causal, forward with P: 40.9 us
    // at 12 chunks, 38.6 at 8; T16384: 104.7 us at 8, 128 at 11).
    const int64_t cfloor = fam == ttt::kFamFwdP ? (lmax + ttt::kLseMergeBatch - 1) / ttt::kLseMergeBatch : 0;
    c = bh * s.nblk >= fill ? lmax : best_chunk(pr, len, col, bh, slots, cfloor);
  }
  s.chunk = (int)std::min<int64_t>(c, lmax);
  s.nchunk_max = (int)((lmax + s.chunk - 1) / s.chunk);
  return s;
}

int family_of(const ttt_problem* pr, int entry, bool gdo) {
  switch (entry) {
    case TTT_ENTRY_FWD:
      return ttt::fwd_row_pairs(pr->dtype, (int)pr->head_dim, has_xm(pr), pr->block_rows) ? ttt::kFamFwdPairs
                                                                                          : ttt::kFamFwdOnline;
    case TTT_ENTRY_FWD_P: return ttt::kFamFwdP;
    case TTT_ENTRY_BWD_DQ: return ttt::kFamDq;
    case TTT_ENTRY_BWD_DKDV: return ttt::kFamDkdv;
    case TTT_ENTRY_GG_ROW: return gdo ? ttt::kFamGgRowGdo : ttt::kFamGgRow;
    case TTT_ENTRY_GG_COL: return ttt::kFamGgCol;
    default: return -1;
  }
}

// Bytes of partial accumulators + partial row scalars for one kernel family.
int64_t family_bytes(const ttt_problem* pr, const Split& s, int fam) {
  if (s.nchunk_max <= 1) return 0;
  const int64_t parts = pr->batch * pr->heads * s.nblk * s.nchunk_max;
  return parts * ttt::kBlk * (ttt::kFamNacc[fam] * pr->head_dim + ttt::kFamNsc[fam]) * (int64_t)sizeof(float);
}

// Workspace of a family: the larger of its two variants' (with and without
// P), since a workspace query does not say which one will run.
int64_t fam_bytes(const ttt_problem* pr, int fam) {
  return std::max(family_bytes(pr, choose_split(pr, fam, false), fam),
                  family_bytes(pr, choose_split(pr, fam, true), fam));
}

int64_t entry_bytes(const ttt_problem* pr, int entry, bool gdo) {
  // the fused backward keeps dQ's partials while dK/dV writes its own
  if (entry == TTT_ENTRY_BWD) return fam_bytes(pr, ttt::kFamDq) + fam_bytes(pr, ttt::kFamDkdv);
  // the fused double backward keeps the row pass's partials while the column
  // pass writes its own
  if (entry == TTT_ENTRY_GG) return fam_bytes(pr, family_of(pr, TTT_ENTRY_GG_ROW, gdo)) + fam_bytes(pr, ttt::kFamGgCol);
  const int fam = family_of(pr, entry, gdo);
  return fam < 0 ? -1 : fam_bytes(pr, fam);
}

ttt::Params base_params(const ttt_problem* pr) {
  ttt::Params a;
  std::memset(&a, 0, sizeof(a));
  a.B = (int)pr->batch;
  a.H = (int)pr->heads;
  a.T = (int)pr->seqlen;
  a.causal = pr->causal;
  a.win = eff_window(pr);
  a.win_kind = pr->window_kind;
  a.bias.p = pr->bias.data;
  a.bias.sb = pr->bias.stride_b;
  a.bias.sh = pr->bias.stride_h;
  a.bias.st = pr->bias.stride_t;
  a.scale = pr->scale;
  a.scale_log2 = pr->scale * ttt::kLog2e;
  return a;
}

// The split of choose_split, with fewer chunks per block if its partials
// would need more than `cap` bytes (cap < 0: no limit).  One chunk per block
// needs none, so some split always fits.
Split capped_split(const ttt_problem* pr, int fam, bool load_p, int64_t cap) {
  Split s = choose_split(pr, fam, load_p);
  if (cap < 0 || family_bytes(pr, s, fam) <= cap) return s;
  const std::vector<int64_t> len = block_tiles(pr, column_family(fam));
  const int64_t lmax = *std::max_element(len.begin(), len.end());
  for (int64_t nch = s.nchunk_max - 1; nch >= 1; --nch) {
    s.chunk = (int)((lmax + nch - 1) / nch);
    s.nchunk_max = (int)((lmax + s.chunk - 1) / s.chunk);
    if (family_bytes(pr, s, fam) <= cap) break;
  }
  return s;
}

// Attach the split and the workspace for kernel family `fam`; the split's
// partials must fit in `cap` bytes (cap < 0: no limit).
int attach_split(const ttt_problem* pr, int fam, bool load_p, void* ws, int64_t ws_bytes, ttt::Params* a,
                 int64_t cap = -1) {
  const Split s = capped_split(pr, fam, load_p, cap);
  a->chunk = s.chunk;
  a->nchunk_max = s.nchunk_max;
  const int64_t need = family_bytes(pr, s, fam);
  if (need > 0) {
    if (!ws || ws_bytes < need)
      return fail(TTT_ERR_WORKSPACE, "workspace of %lld bytes needed, %lld given", (long long)need,
                  (long long)(ws ? ws_bytes : 0));
    if (!aligned16(ws)) return fail(TTT_ERR_INVALID_ARGUMENT, "workspace not 16-byte aligned");
    const int64_t parts = pr->batch * pr->heads * s.nblk * s.nchunk_max;
    a->ws_acc = reinterpret_cast<float*>(ws);
    a->ws_sc = a->ws_acc + parts * ttt::kBlk * ttt::kFamNacc[fam] * pr->head_dim;
  }
  return TTT_OK;
}

bool has_p(const ttt_view* p) { return p && p->data; }

// Row-statistic arrays (lse, rowsum, E, F) must be 16-byte aligned.
int check_stats(std::initializer_list<const void*> ptrs) {
  for (const void* q : ptrs)
    if (q && !aligned16(q)) return fail(TTT_ERR_INVALID_ARGUMENT, "row-statistic array not 16-byte aligned");
  return TTT_OK;
}

int launched(hipError_t e, const char* what) {
  if (e != hipSuccess) return fail(TTT_ERR_LAUNCH, "%s: launch failed: %s", what, hipGetErrorString(e));
  return TTT_OK;
}

#define TRY(x)                     \
  do {                             \
    const int rc_ = (x);           \
    if (rc_ != TTT_OK) return rc_; \
  } while (0)

}  // namespace

// ---------------------------------------------------------------------------
// Scratch of the entry point that allocates nothing (ttt_attn_gg_noalloc):
// its E and F row statistics, then the partial sums of its split.  A
// file-scope device array, so every GPU the library runs on holds its own
// copy from module load until the process ends.  Host code never uses the
// array's name as an address (on the host it is only a stand-in): the first
// call on a device looks up that device's copy with hipGetSymbolAddress and
// keeps the pointer.  Calls on one GPU share its copy, so calls that overlap
// on one GPU (different streams, or threads) race; nothing in it needs to
// start at zero (every kernel writes what it later reads).
constexpr int64_t kNoAllocScratchBytes = 64ll << 20;
constexpr int64_t kNoAllocStatBytes = 16ll << 20;  // E and F: B*H*T <= 2^21
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

namespace {

constexpr int kMaxDevices = 64;

// This device's copy of `scratch` (looked up once per device).
int scratch_on_device(void** out) {
  static std::mutex mu;
  static void* ptr[kMaxDevices] = {};
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail(TTT_ERR_LAUNCH, "hipGetDevice: %s", hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices) return fail(TTT_ERR_UNSUPPORTED, "device %d: at most %d devices", dev, kMaxDevices);
  std::lock_guard<std::mutex> lock(mu);
  if (!ptr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return fail(TTT_ERR_LAUNCH, "hipGetSymbolAddress(scratch) on device %d: %s", dev, hipGetErrorString(e));
    ptr[dev] = p;
  }
  *out = ptr[dev];
  return TTT_OK;
}

// Per-kernel timing (ttt_kernel_timing): a pool of HIP events, two per timed
// launch, recorded in launch order with their kernel tag.  Used from one host
// thread at a time, as the ABI documents.
struct TimingPool {
  std::vector<hipEvent_t> ev;  // pairs: event 2i starts launch i, event 2i + 1 ends it
  std::vector<int> tag;        // per event: the launch's kernel tag
  int used = 0;
  bool on = false;
  bool open = false;  // a start is recorded and its end is not
};
TimingPool g_timing;

}  // namespace

namespace ttt {
void timing_mark(hipStream_t st, int tag, bool end) {
  TimingPool& t = g_timing;
  if (!t.on || end != t.open) return;
  if (end && t.tag[t.used - 1] != tag) return;
  if (!end && t.used + 2 > (int)t.ev.size()) return;  // room for the pair
  if (hipEventRecord(t.ev[t.used], st) != hipSuccess) {
    (void)hipGetLastError();
    if (end) {  // drop the unmatched start
      --t.used;
      t.open = false;
    }
    return;
  }
  t.tag[t.used++] = tag;
  t.open = !end;
}
}  // namespace ttt

extern "C" {

int ttt_version(void) { return 400; }

int ttt_kernel_timing(int32_t capacity) {
  TimingPool& t = g_timing;
  t.on = false;
  t.open = false;
  t.used = 0;
  if (capacity <= 0) return TTT_OK;
  if (capacity > (1 << 16)) return fail(TTT_ERR_INVALID_ARGUMENT, "kernel_timing: capacity %d > 65536", capacity);
  while ((int)t.ev.size() < 2 * capacity) {
    hipEvent_t e;
    if (hipEventCreate(&e) != hipSuccess) {
      (void)hipGetLastError();
      return fail(TTT_ERR_LAUNCH, "kernel_timing: hipEventCreate failed");
    }
    t.ev.push_back(e);
    t.tag.push_back(-1);
  }
  t.on = true;
  return TTT_OK;
}

int ttt_kernel_timing_read(int32_t kernel, float* mean_ms, int32_t* count) {
  if (kernel < 0 || kernel >= ttt::kNumTags) return fail(TTT_ERR_INVALID_ARGUMENT, "kernel_timing_read: kernel %d", kernel);
  TimingPool& t = g_timing;
  double sum = 0.0;
  int n = 0;
  for (int i = 0; i + 1 < t.used; i += 2) {
    if (t.tag[i] != kernel) continue;
    float ms = 0.f;
    if (hipEventSynchronize(t.ev[i + 1]) != hipSuccess || hipEventElapsedTime(&ms, t.ev[i], t.ev[i + 1]) != hipSuccess) {
      (void)hipGetLastError();
      return fail(TTT_ERR_LAUNCH, "kernel_timing_read: event %d", i);
    }
    sum += ms;
    ++n;
  }
  if (mean_ms) *mean_ms = n ? (float)(sum / n) : 0.f;
  if (count) *count = n;
  return TTT_OK;
}

const char* ttt_last_error(void) { return g_err; }

int64_t ttt_attn_workspace_size(const ttt_problem* pr, int32_t entry, int32_t want_gdout) {
  if (check_problem(pr) != TTT_OK) return -1;
  if (entry < TTT_ENTRY_FWD || entry > TTT_ENTRY_GG) {
    fail(TTT_ERR_INVALID_ARGUMENT, "unknown entry %d", entry);
    return -1;
  }
  return entry_bytes(pr, entry, want_gdout != 0);
}

int ttt_attn_split_info(const ttt_problem* pr, int32_t entry, int32_t load_p, int32_t want_gdout, int32_t* chunk,
                        int32_t* nchunk_max, int64_t* slots) {
  TRY(check_problem(pr));
  const int fam = family_of(pr, entry, want_gdout != 0);
  if (fam < 0) return fail(TTT_ERR_INVALID_ARGUMENT, "entry %d is not a single kernel family", entry);
  const Split s = choose_split(pr, fam, load_p != 0);
  if (chunk) *chunk = s.chunk;
  if (nchunk_max) *nchunk_max = s.nchunk_max;
  if (slots) *slots = family_slots(pr, fam, load_p != 0);
  return TTT_OK;
}

int ttt_attn_launch_item(int32_t nblk, int32_t chunk, int32_t column, int32_t* block, int32_t* chunk_index) {
  if (nblk <= 0 || chunk <= 0 || column < 0 || (int64_t)column >= (int64_t)nblk * ((nblk + chunk - 1) / chunk))
    return fail(TTT_ERR_INVALID_ARGUMENT, "launch_item: nblk %d, chunk %d, column %d", nblk, chunk, column);
  const ttt::Item it = ttt::causal_item(column, nblk, chunk);
  if (block) *block = it.blk;
  if (chunk_index) *chunk_index = it.ch;
  return TTT_OK;
}

int ttt_attn_fwd(const ttt_problem* pr, const ttt_view* q, const ttt_view* k, const ttt_view* v,
                 const ttt_view* o, float* lse, const ttt_view* p, void* workspace, int64_t workspace_bytes,
                 void* stream) {
  TRY(check_problem(pr));
  ttt::Params a = base_params(pr);
  TRY(take_view(pr, q, "q", &a.q));
  TRY(take_view(pr, k, "k", &a.k));
  TRY(take_view(pr, v, "v", &a.v));
  TRY(take_view(pr, o, "o", &a.o));
  if (!lse) return fail(TTT_ERR_INVALID_ARGUMENT, "lse: null pointer");
  TRY(check_stats({lse}));
  a.lse = lse;
  const bool wp = has_p(p);
  if (wp) TRY(take_view(pr, p, "p", &a.p));
  if (!wp && pr->block_rows == 128 && !ttt::fwd_pairs_allowed(pr->dtype, has_xm(pr)))
    return fail(TTT_ERR_UNSUPPORTED, "block_rows 128: 16-bit types without a window or bias only");
  const int fam = wp ? ttt::kFamFwdP : family_of(pr, TTT_ENTRY_FWD, false);
  a.pairs = fam == ttt::kFamFwdPairs ? 1 : 0;
  TRY(attach_split(pr, fam, wp, workspace, workspace_bytes, &a));
  // Deferred P stores pay off where the P writes run at bandwidth: several
  // rounds of workgroups per slot (b4 h16 T8192 d128: P pass -11 %); with one
  // round they cost about 1 % (b2 h4 T2048 d128).
  if (wp) {
    const int64_t blocks = pr->batch * pr->heads * ((pr->seqlen + ttt::kBlk - 1) / ttt::kBlk);
    a.defer_p = blocks >= kDeferRounds * family_slots(pr, ttt::kFamFwdP, true) ? 1 : 0;
    const int64_t written = pr->batch * pr->heads * pr->seqlen * pr->seqlen * (pr->dtype == TTT_F32 ? 4 : 2) /
                            (pr->causal ? 2 : 1);
    a.p_nt = written > kPStreamBytes ? 1 : 0;
  }
  return launched(ttt::launch_fwd(pr->dtype, (int)pr->head_dim, a, wp, (hipStream_t)stream), "ttt_attn_fwd");
}

int ttt_attn_fill_masked_p(const ttt_problem* pr, const ttt_view* p, void* stream) {
  TRY(check_problem(pr));
  ttt::Params a = base_params(pr);
  TRY(take_view(pr, p, "p", &a.p));
  return launched(ttt::launch_fill_masked_p(pr->dtype, a, (hipStream_t)stream), "ttt_attn_fill_masked_p");
}

}  // extern "C"

// Parameters of the dQ launch (ttt_attn_bwd_dq), its split and workspace.
static int prep_dq(const ttt_problem* pr, const ttt_view* q, const ttt_view* k, const ttt_view* v,
                   const ttt_view* o, const ttt_view* dout, const float* lse, const ttt_view* p, const float* rowsum_in,
                   float* rowsum_out, const ttt_view* dq, void* workspace, int64_t workspace_bytes, ttt::Params* out) {
  TRY(check_problem(pr));
  ttt::Params a = base_params(pr);
  TRY(take_view(pr, k, "k", &a.k));
  TRY(take_view(pr, v, "v", &a.v));
  TRY(take_view(pr, dout, "dout", &a.dout));
  TRY(take_view(pr, dq, "dq", &a.dq));
  const bool lp = has_p(p);
  if (lp) {
    TRY(take_view(pr, p, "p", &a.p));
  } else {
    TRY(take_view(pr, q, "q", &a.q));
    if (!lse) return fail(TTT_ERR_INVALID_ARGUMENT, "lse: null pointer (required without p)");
  }
  TRY(check_stats({lse, rowsum_in, rowsum_out}));
  a.lse = const_cast<float*>(lse);
  a.rowsum_in = rowsum_in;
  a.rowsum_out = rowsum_out;
  if (!rowsum_in) TRY(take_view(pr, o, "o (needed to form D without rowsum_in)", &a.o));
  TRY(attach_split(pr, ttt::kFamDq, lp, workspace, workspace_bytes, &a));
  *out = a;
  return TTT_OK;
}

// Parameters of the dK/dV launch (ttt_attn_bwd_dkdv), its split and workspace.
static int prep_dkdv(const ttt_problem* pr, const ttt_view* q, const ttt_view* k, const ttt_view* v,
                     const ttt_view* dout, const float* lse, const ttt_view* p, const float* rowsum,
                     const ttt_view* dk, const ttt_view* dv, void* workspace, int64_t workspace_bytes,
                     ttt::Params* out) {
  TRY(check_problem(pr));
  ttt::Params a = base_params(pr);
  const bool lp = has_p(p);
  const bool dv_only = !(dk && dk->data);
  TRY(take_view(pr, dout, "dout", &a.dout));
  TRY(take_view(pr, dv, "dv", &a.dv));
  if (lp) TRY(take_view(pr, p, "p", &a.p));
  if (!lp) {
    TRY(take_view(pr, k, "k", &a.k));
    if (!lse) return fail(TTT_ERR_INVALID_ARGUMENT, "lse: null pointer (required without p)");
  }
  if (!lp || !dv_only) TRY(take_view(pr, q, "q", &a.q));
  if (!dv_only) {
    TRY(take_view(pr, v, "v", &a.v));
    TRY(take_view(pr, dk, "dk", &a.dk));
    if (!rowsum) return fail(TTT_ERR_INVALID_ARGUMENT, "rowsum: null pointer (required for dk)");
  }
  TRY(check_stats({lse, rowsum}));
  a.lse = const_cast<float*>(lse);
  a.rowsum_in = rowsum;
  TRY(attach_split(pr, ttt::kFamDkdv, lp, workspace, workspace_bytes, &a));
  *out = a;
  return TTT_OK;
}

extern "C" {

int ttt_attn_bwd_dq(const ttt_problem* pr, const ttt_view* q, const ttt_view* k, const ttt_view* v,
                    const ttt_view* o, const ttt_view* dout, const float* lse, const ttt_view* p,
                    const float* rowsum_in, float* rowsum_out, const ttt_view* dq, void* workspace,
                    int64_t workspace_bytes, void* stream) {
  ttt::Params a;
  TRY(prep_dq(pr, q, k, v, o, dout, lse, p, rowsum_in, rowsum_out, dq, workspace, workspace_bytes, &a));
  return launched(ttt::launch_bwd_dq(pr->dtype, (int)pr->head_dim, a, has_p(p), (hipStream_t)stream),
                  "ttt_attn_bwd_dq");
}

int ttt_attn_bwd_dkdv(const ttt_problem* pr, const ttt_view* q, const ttt_view* k, const ttt_view* v,
                      const ttt_view* dout, const float* lse, const ttt_view* p, const float* rowsum,
                      const ttt_view* dk, const ttt_view* dv, void* workspace, int64_t workspace_bytes,
                      void* stream) {
  ttt::Params a;
  TRY(prep_dkdv(pr, q, k, v, dout, lse, p, rowsum, dk, dv, workspace, workspace_bytes, &a));
  const bool dv_only = !(dk && dk->data);
  return launched(ttt::launch_bwd_dkdv(pr->dtype, (int)pr->head_dim, a, has_p(p), dv_only, (hipStream_t)stream),
                  "ttt_attn_bwd_dkdv");
}

// dQ's partials go in the first part of the workspace and dK/dV's after them:
// the dK/dV launch sums dQ's split blocks in workgroups appended to its grid
// while its own blocks write their partials.
int ttt_attn_bwd(const ttt_problem* pr, const ttt_view* q, const ttt_view* k, const ttt_view* v,
                 const ttt_view* o, const ttt_view* dout, const float* lse, const ttt_view* p,
                 float* rowsum_out, const ttt_view* dq, const ttt_view* dk, const ttt_view* dv,
                 void* workspace, int64_t workspace_bytes, void* stream) {
  if (!rowsum_out) return fail(TTT_ERR_INVALID_ARGUMENT, "rowsum_out: null pointer");
  if (!dk || !dk->data) return fail(TTT_ERR_INVALID_ARGUMENT, "dk: null pointer");
  TRY(check_problem(pr));
  const bool lp = has_p(p);
  const int64_t dq_bytes = family_bytes(pr, choose_split(pr, ttt::kFamDq, lp), ttt::kFamDq);
  const int64_t ws_bytes = workspace ? workspace_bytes : 0;
  ttt::Params aq, ak;
  TRY(prep_dq(pr, q, k, v, o, dout, lse, p, nullptr, rowsum_out, dq, workspace, ws_bytes, &aq));
  if (ws_bytes < dq_bytes)  // prep_dq has checked this; kept for the pointer arithmetic below
    return fail(TTT_ERR_WORKSPACE, "workspace of %lld bytes too small", (long long)ws_bytes);
  void* ws_k = dq_bytes > 0 ? static_cast<void*>(static_cast<char*>(workspace) + dq_bytes) : workspace;
  TRY(prep_dkdv(pr, q, k, v, dout, lse, p, rowsum_out, dk, dv, ws_k, ws_bytes - dq_bytes, &ak));
  const hipStream_t st = (hipStream_t)stream;
  TRY(launched(ttt::launch_bwd_dq(pr->dtype, (int)pr->head_dim, aq, lp, st, false), "ttt_attn_bwd"));
  return launched(ttt::launch_bwd_dkdv(pr->dtype, (int)pr->head_dim, ak, lp, false, st, &aq), "ttt_attn_bwd");
}

int ttt_attn_bwd_rowsum(const ttt_problem* pr, const ttt_view* p, const ttt_view* dout, const ttt_view* v,
                        float* rowsum, void* stream) {
  TRY(check_problem(pr));
  ttt::Params a = base_params(pr);
  TRY(take_view(pr, p, "p", &a.p));
  TRY(take_view(pr, dout, "dout", &a.dout));
  TRY(take_view(pr, v, "v", &a.v));
  if (!rowsum) return fail(TTT_ERR_INVALID_ARGUMENT, "rowsum: null pointer");
  TRY(check_stats({rowsum}));
  a.rowsum_out = rowsum;
  return launched(ttt::launch_bwd_rowsum(pr->dtype, (int)pr->head_dim, a, (hipStream_t)stream),
                  "ttt_attn_bwd_rowsum");
}

// ttt_attn_gg_row / ttt_attn_gg_col with the split's partials held to `cap`
// bytes (cap < 0: no limit).
static int prep_gg_row(const ttt_problem* pr, const ttt_view* q, const ttt_view* k, const ttt_view* v,
                       const ttt_view* dout, const float* lse, const ttt_view* p, const float* rowsum,
                       const ttt_view* dq, const ttt_view* gq, const ttt_view* gk, const ttt_view* gv,
                       const ttt_view* gq_out,
                       const ttt_view* gdout, float* e_out, float* f_out, void* workspace, int64_t workspace_bytes,
                       int64_t cap, ttt::Params* out) {
  TRY(check_problem(pr));
  ttt::Params a = base_params(pr);
  TRY(take_view(pr, q, "q", &a.q));
  TRY(take_view(pr, k, "k", &a.k));
  TRY(take_view(pr, v, "v", &a.v));
  TRY(take_view(pr, dout, "dout", &a.dout));
  TRY(take_view(pr, gq, "gq", &a.gq));
  TRY(take_view(pr, gk, "gk", &a.gk));
  TRY(take_view(pr, gv, "gv", &a.gv));
  TRY(take_view(pr, gq_out, "gq_out", &a.gq_out));
  const bool lp = has_p(p);
  if (lp) TRY(take_view(pr, p, "p", &a.p));
  if (!lp && !lse) return fail(TTT_ERR_INVALID_ARGUMENT, "lse: null pointer (required without p)");
  const bool gdo = gdout && gdout->data;
  if (gdo) TRY(take_view(pr, gdout, "gdout", &a.gdout));
  // the first backward's dQ: read by the row pass without GdO (the kernels
  // and combines take a.dq.p set as the dQ form)
  if (dq && dq->data && !gdo) TRY(take_view(pr, dq, "dq", &a.dq));
  if (!rowsum || !e_out || !f_out) return fail(TTT_ERR_INVALID_ARGUMENT, "rowsum/e_out/f_out: null pointer");
  TRY(check_stats({lse, rowsum, e_out, f_out}));
  a.lse = const_cast<float*>(lse);
  a.rowsum_in = rowsum;
  a.e = e_out;
  a.f = f_out;
  TRY(attach_split(pr, gdo ? ttt::kFamGgRowGdo : ttt::kFamGgRow, lp, workspace, workspace_bytes, &a, cap));
  *out = a;
  return TTT_OK;
}

static int gg_row_impl(const ttt_problem* pr, const ttt_view* q, const ttt_view* k, const ttt_view* v,
                       const ttt_view* dout, const float* lse, const ttt_view* p, const float* rowsum,
                       const ttt_view* dq, const ttt_view* gq, const ttt_view* gk, const ttt_view* gv,
                       const ttt_view* gq_out, const ttt_view* gdout, float* e_out, float* f_out, void* workspace,
                       int64_t workspace_bytes, void* stream, int64_t cap) {
  ttt::Params a;
  TRY(prep_gg_row(pr, q, k, v, dout, lse, p, rowsum, dq, gq, gk, gv, gq_out, gdout, e_out, f_out, workspace,
                  workspace_bytes, cap, &a));
  return launched(ttt::launch_gg_row(pr->dtype, (int)pr->head_dim, a, has_p(p), a.gdout.p != nullptr,
                                     (hipStream_t)stream),
                  "ttt_attn_gg_row");
}

static int prep_gg_col(const ttt_problem* pr, const ttt_view* q, const ttt_view* k, const ttt_view* v,
                       const ttt_view* dout, const float* lse, const ttt_view* p, const float* rowsum,
                       const float* e_in, const float* f_in, const ttt_view* gq, const ttt_view* gk,
                       const ttt_view* gv, const ttt_view* gk_out, const ttt_view* gv_out, void* workspace,
                       int64_t workspace_bytes, int64_t cap, ttt::Params* out) {
  TRY(check_problem(pr));
  ttt::Params a = base_params(pr);
  TRY(take_view(pr, q, "q", &a.q));
  TRY(take_view(pr, k, "k", &a.k));
  TRY(take_view(pr, v, "v", &a.v));
  TRY(take_view(pr, dout, "dout", &a.dout));
  TRY(take_view(pr, gq, "gq", &a.gq));
  TRY(take_view(pr, gk, "gk", &a.gk));
  TRY(take_view(pr, gv, "gv", &a.gv));
  TRY(take_view(pr, gk_out, "gk_out", &a.gk_out));
  TRY(take_view(pr, gv_out, "gv_out", &a.gv_out));
  const bool lp = has_p(p);
  if (lp) TRY(take_view(pr, p, "p", &a.p));
  if (!lp && !lse) return fail(TTT_ERR_INVALID_ARGUMENT, "lse: null pointer (required without p)");
  if (!rowsum || !e_in || !f_in) return fail(TTT_ERR_INVALID_ARGUMENT, "rowsum/e_in/f_in: null pointer");
  TRY(check_stats({lse, rowsum, e_in, f_in}));
  a.lse = const_cast<float*>(lse);
  a.rowsum_in = rowsum;
  a.e = const_cast<float*>(e_in);
  a.f = const_cast<float*>(f_in);
  TRY(attach_split(pr, ttt::kFamGgCol, lp, workspace, workspace_bytes, &a, cap));
  *out = a;
  return TTT_OK;
}

static int gg_col_impl(const ttt_problem* pr, const ttt_view* q, const ttt_view* k, const ttt_view* v,
                       const ttt_view* dout, const float* lse, const ttt_view* p, const float* rowsum,
                       const float* e_in, const float* f_in, const ttt_view* gq, const ttt_view* gk,
                       const ttt_view* gv, const ttt_view* gk_out, const ttt_view* gv_out, void* workspace,
                       int64_t workspace_bytes, void* stream, int64_t cap) {
  ttt::Params a;
  TRY(prep_gg_col(pr, q, k, v, dout, lse, p, rowsum, e_in, f_in, gq, gk, gv, gk_out, gv_out, workspace,
                  workspace_bytes, cap, &a));
  return launched(ttt::launch_gg_col(pr->dtype, (int)pr->head_dim, a, has_p(p), (hipStream_t)stream),
                  "ttt_attn_gg_col");
}

int ttt_attn_gg_row(const ttt_problem* pr, const ttt_view* q, const ttt_view* k, const ttt_view* v,
                    const ttt_view* dout, const float* lse, const ttt_view* p, const float* rowsum,
                    const ttt_view* dq, const ttt_view* gq, const ttt_view* gk, const ttt_view* gv,
                    const ttt_view* gq_out, const ttt_view* gdout, float* e_out, float* f_out, void* workspace,
                    int64_t workspace_bytes, void* stream) {
  return gg_row_impl(pr, q, k, v, dout, lse, p, rowsum, dq, gq, gk, gv, gq_out, gdout, e_out, f_out, workspace,
                     workspace_bytes, stream, -1);
}

int ttt_attn_gg_col(const ttt_problem* pr, const ttt_view* q, const ttt_view* k, const ttt_view* v,
                    const ttt_view* dout, const float* lse, const ttt_view* p, const float* rowsum,
                    const float* e_in, const float* f_in, const ttt_view* gq, const ttt_view* gk,
                    const ttt_view* gv, const ttt_view* gk_out, const ttt_view* gv_out, void* workspace,
                    int64_t workspace_bytes, void* stream) {
  return gg_col_impl(pr, q, k, v, dout, lse, p, rowsum, e_in, f_in, gq, gk, gv, gk_out, gv_out, workspace,
                     workspace_bytes, stream, -1);
}

int ttt_attn_gg(const ttt_problem* pr, const ttt_view* q, const ttt_view* k, const ttt_view* v,
                const ttt_view* dout, const float* lse, const ttt_view* p, const float* rowsum,
                const ttt_view* dq, const ttt_view* gq, const ttt_view* gk, const ttt_view* gv,
                const ttt_view* gq_out, const ttt_view* gk_out, const ttt_view* gv_out, const ttt_view* gdout,
                float* e_buf, float* f_buf, void* workspace, int64_t workspace_bytes, void* stream) {
  // The row pass's partials go in the first part of the workspace and the
  // column pass's after them: the column launch sums the row pass's split
  // blocks (GQ, GdO) in workgroups appended to its grid, after a small launch
  // has formed E and F, which the column pass reads.
  TRY(check_problem(pr));
  const bool lp = has_p(p);
  const bool gdo = gdout && gdout->data;
  const int fam = gdo ? ttt::kFamGgRowGdo : ttt::kFamGgRow;
  const int64_t row_bytes = family_bytes(pr, choose_split(pr, fam, lp), fam);
  const int64_t ws_bytes = workspace ? workspace_bytes : 0;
  ttt::Params ar, ac;
  TRY(prep_gg_row(pr, q, k, v, dout, lse, p, rowsum, dq, gq, gk, gv, gq_out, gdout, e_buf, f_buf, workspace,
                  ws_bytes, -1, &ar));
  if (ws_bytes < row_bytes)  // prep_gg_row has checked this; kept for the pointer arithmetic below
    return fail(TTT_ERR_WORKSPACE, "workspace of %lld bytes too small", (long long)ws_bytes);
  void* ws_c = row_bytes > 0 ? static_cast<void*>(static_cast<char*>(workspace) + row_bytes) : workspace;
  TRY(prep_gg_col(pr, q, k, v, dout, lse, p, rowsum, e_buf, f_buf, gq, gk, gv, gk_out, gv_out, ws_c,
                  ws_bytes - row_bytes, -1, &ac));
  const hipStream_t st = (hipStream_t)stream;
  TRY(launched(ttt::launch_gg_row(pr->dtype, (int)pr->head_dim, ar, lp, gdo, st, false), "ttt_attn_gg"));
  return launched(ttt::launch_gg_col(pr->dtype, (int)pr->head_dim, ac, lp, st, &ar), "ttt_attn_gg");
}

int ttt_attn_gg_noalloc(const ttt_problem* pr, const ttt_view* q, const ttt_view* k, const ttt_view* v,
                        const ttt_view* dout, const float* lse, const ttt_view* p, const float* rowsum,
                        const ttt_view* dq, const ttt_view* gq, const ttt_view* gk, const ttt_view* gv,
                        const ttt_view* gq_out, const ttt_view* gk_out, const ttt_view* gv_out,
                        const ttt_view* gdout, void* stream) {
  TRY(check_problem(pr));
  const int64_t nstat = pr->batch * pr->heads * pr->seqlen;
  const int64_t one = (nstat * (int64_t)sizeof(float) + 255) / 256 * 256;  // E, then F, 256-byte aligned
  if (2 * one > kNoAllocStatBytes)
    return fail(TTT_ERR_INVALID_ARGUMENT,
                "ttt_attn_gg_noalloc: B*H*T = %lld needs %lld bytes of E/F statistics, more than the %lld its "
                "scratch holds (B*H*T <= %lld); use ttt_attn_gg with caller buffers",
                (long long)nstat, (long long)(2 * one), (long long)kNoAllocStatBytes,
                (long long)(kNoAllocStatBytes / 8));
  void* base = nullptr;
  TRY(scratch_on_device(&base));
  float* e = static_cast<float*>(base);
  float* f = reinterpret_cast<float*>(static_cast<char*>(base) + one);
  void* ws = static_cast<char*>(base) + 2 * one;
  const int64_t ws_bytes = kNoAllocScratchBytes - 2 * one;
  TRY(gg_row_impl(pr, q, k, v, dout, lse, p, rowsum, dq, gq, gk, gv, gq_out, gdout, e, f, ws, ws_bytes, stream,
                  ws_bytes));
  return gg_col_impl(pr, q, k, v, dout, lse, p, rowsum, e, f, gq, gk, gv, gk_out, gv_out, ws, ws_bytes, stream,
                     ws_bytes);
}

}  // extern "C"
