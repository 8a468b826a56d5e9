// ttt_bwd.hip — first backward of attention for gfx950.
//
//   k_bwd_dq    row-block kernel (stationary query rows m, streamed key tiles):
//               dP^T = V*dO^T, dS = P o (dP - D), dQ^T += K^T*dS^T.
//               Prologue: D[m] = rowsum(dO o O)[m] unless supplied.
//   k_bwd_dkdv  column-block kernel (stationary key rows n, streamed query
//               tiles): dV^T += dO^T*P, dP = dO*V^T, dS = P o (dP - D),
//               dK^T += Q^T*dS.
//   k_bwd_rowsum  row-block kernel for rowsum[m] = sum_n P*(dO*V^T), the
//               reference's definition of the row statistic from P.
//
// LOADP = true reads P from the [B,H,T,T] matrix written by the forward (row
// kernels load the lane's 8-element row fragments straight from HBM; column
// kernels stage the 64x64 P tile in LDS and read it by columns);
// LOADP = false recomputes P = exp2(s*log2e*QK^T - lse*log2e) per tile.
// Causal: fully masked tiles are skipped, diagonal tiles masked per element;
// a key window likewise (RowMask / ColMask).  Recomputed P adds the additive
// bias when there is one (saved P already holds it).  XM instantiates the
// window/bias code.
// The next tile's loads are issued before the current tile's math.
// dP - D comes out of the MFMAs: in k_bwd_dq they start from -D (the
// stationary row's), in k_bwd_dkdv from the streamed rows' D with the
// stationary V fragments negated (then D - dP, and dK is stored negated back).
//
// Reference semantics: ttt_kernels/triton_attention.py:364-378 (save_p torch
// backward), :416-420 (recompute); ttt_kernels/backward_stubs.py:124-425.
#include "ttt_combine.h"

// Fetch forms, measured on MI355X and kept:
//  * 16-bit tiles stream into LDS by direct loads: the saved-P dQ kernel's
//    key tiles (D = 64: two buffers of one array picked at run time, which
//    measured 3-12 % faster than two sets in distinct arrays; D = 128: two
//    sets with compile-time roles), and the recompute dQ kernel's K and V
//    (D = 64, two sets).
//  * Register-staged dQ tiles: full tiles through per-lane offsets computed
//    once (else stage_load's clamped addressing), and the last tile peeled
//    off the loop so the next tile's fetch inside it is unconditional (its
//    registers then need no copies across iterations).  In dK/dV both forms
//    cost registers (up to +24 VGPRs, past an occupancy step at D = 128:
//    b4 h16 T8192 dK/dV +20 %), so dK/dV stages with clamped addressing and
//    no peeled tile.
//  * The saved-P dK/dV kernel streams 16-bit tiles by direct loads into two
//    buffer sets: dO, Q, P and the rowsum slice at D = 64; dO, Q and the
//    rowsum slice at D = 128, with P staged through registers.  The
//    recompute dK/dV kernel (16-bit, D = 64) streams dO, Q and its two row
//    statistics the same way.

namespace ttt {

// D for this lane's row from the lane's dO fragments and O read in the same
// layout.
template <typename T, int D>
__device__ __forceinline__ float row_dot_do_o(const typename Elem<T>::frag* dof, const T* O, int64_t ld,
                                              int m, int T_) {
  const int g = (threadIdx.x & 63) >> 4;
  float acc = 0.f;
#pragma unroll
  for (int ks = 0; ks < D / 32; ++ks) {
    const typename Elem<T>::frag of = load_frag_row<T>(O, ld, m, T_, 32 * ks + 8 * g);
#pragma unroll
    for (int j = 0; j < 8; ++j) acc += Elem<T>::f32(dof[ks][j]) * Elem<T>::f32(of[j]);
  }
  return group_sum(acc);
}

template <typename T>
__device__ __forceinline__ void frags_to_tile(Tile& p, const typename Elem<T>::frag* f) {
#pragma unroll
  for (int kb = 0; kb < 2; ++kb)
#pragma unroll
    for (int j = 0; j < 8; ++j) p.set(kb, j, Elem<T>::f32(f[kb][j]));
}

// Waves per EU the dQ kernel is compiled for: VGPR accumulators (AccWaves)
// for the D = 64 recompute variants, and for their 16-bit types a cap of 128
// registers, which keeps four waves per SIMD (the window/bias variant sits
// right at that boundary; at 132 registers it drops to three, measured
// b8 h6 T8192 d64 bf16 local window 512: dQ 101 -> 113 us).
template <typename T, int D, bool LOADP>
struct DqWaves {
  static constexpr bool kVacc = !LOADP && D == 64;
  // The saved-P 16-bit D = 128 kernel in the two-set form (two tiles per loop
  // step): without a register cap the compiler keeps the accumulators in
  // AGPRs and copies them every step.
  static constexpr bool kPar = LOADP && sizeof(T) == 2 && D == 128;
  static constexpr int value =
      kVacc ? (sizeof(T) == 2 ? 4 : AccWaves<true>::value) : kPar ? (D == 64 ? 3 : 2) : AccWaves<false>::value;
};

// ---------------------------------------------------------------------------
template <typename T, int D, bool LOADP, bool XM>
__global__ __launch_bounds__(kThreads)
__attribute__((amdgpu_waves_per_eu(DqWaves<T, D, LOADP>::value))) void k_bwd_dq(Params a) {
  typedef Elem<T> E;
  typedef typename E::frag frag;
  typedef Lds<T, D> L;
  // Saved-P 16-bit tiles stream straight into two LDS buffers per operand
  // (TileDma): with kPar, two sets in distinct arrays with a compile-time role
  // per loop step (so that the current tile's LDS reads need not wait for the
  // next tile's loads), else two buffers of one array picked at run time.
  constexpr bool kDma = L::kSwizzle && (LOADP || D == 64);
  constexpr bool kPar = kDma && (D == 128 || !LOADP);
  constexpr bool kRt = kDma && !kPar;
  constexpr int kE1 = kPar ? L::kRowElems : 8, kER = kRt ? L::kRowElems : 8;
  __shared__ __align__(16) T sK0[kRt ? 8 : L::kRowElems];
  __shared__ __align__(16) T sV0[kRt ? 8 : L::kRowElems];
  __shared__ __align__(16) T sK1[kE1];
  __shared__ __align__(16) T sV1[kE1];
  __shared__ __align__(16) T sKr[kRt ? 2 : 1][kER];
  __shared__ __align__(16) T sVr[kRt ? 2 : 1][kER];
  auto set_k = [&](auto par) __attribute__((always_inline)) -> T* {
    if constexpr (std::is_same_v<decltype(par), RtBuf>) return sKr[par.cur];
    else if constexpr (decltype(par)::value == 0) return sK0;
    else return sK1;
  };
  auto set_v = [&](auto par) __attribute__((always_inline)) -> T* {
    if constexpr (std::is_same_v<decltype(par), RtBuf>) return sVr[par.cur];
    else if constexpr (decltype(par)::value == 0) return sV0;
    else return sV1;
  };

  const int T_ = a.T;
  const int nblk = (T_ + kBlk - 1) / kBlk;
  const Slot sl = grid_slot();
  const Item it = launch_item<XM>(a, sl.x, nblk);
  if (it.blk < 0) return;
  const int bi = it.blk, ch = it.ch;
  const int bh = sl.y, b = bh / a.H, h = bh % a.H;
  const int mb = a.causal ? (nblk - 1 - bi) : bi;
  const Range rg = row_block_range(mb, nblk, T_, a.causal, XM ? a.win : 0, a.win_kind);
  const Chunk cr = chunk_of(rg.lo, rg.hi, ch, a.chunk);
  if (ch >= cr.nch) return;
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63, c = lane & 15, g = lane >> 4;
  const int rl = 16 * w + c;
  const int m = mb * kBlk + rl;
  const bool row_ok = m < T_;
  const RowMask<XM> mk(a, mb, m);
  const T* brow =
      (XM && !LOADP && a.bias.p) ? at<const T>(a.bias, b, h) + (int64_t)(row_ok ? m : 0) * a.bias.st : nullptr;

  const T* Q = at<const T>(a.q, b, h);
  const T* K = at<const T>(a.k, b, h);
  const T* V = at<const T>(a.v, b, h);
  const T* dO = at<const T>(a.dout, b, h);

  frag dof[D / 32], qf[D / 32];
#pragma unroll
  for (int ks = 0; ks < D / 32; ++ks) {
    dof[ks] = load_frag_row<T>(dO, a.dout.st, m, T_, 32 * ks + 8 * g);
    if constexpr (!LOADP) qf[ks] = load_frag_row<T>(Q, a.q.st, m, T_, 32 * ks + 8 * g);
  }
  const int64_t ridx = (int64_t)bh * T_ + m;
  float Dm;
  if (a.rowsum_in) {
    Dm = row_ok ? a.rowsum_in[ridx] : 0.f;
  } else {
    Dm = row_dot_do_o<T, D>(dof, at<const T>(a.o, b, h), a.o.st, m, T_);
    if (a.rowsum_out && ch == 0 && row_ok && g == 0) a.rowsum_out[ridx] = Dm;
  }
  const f32x4 mDm4 = f32x4{-Dm, -Dm, -Dm, -Dm};  // dP's MFMAs start from -D: they give dP - D
  const float lse2 = (!LOADP && row_ok) ? a.lse[ridx] * kLog2e : 0.f;
  const T* Pm = LOADP ? at<const T>(a.p, b, h) + (int64_t)(row_ok ? m : 0) * a.p.st : nullptr;

  f32x4 acc[D / 16];
#pragma unroll
  for (int i = 0; i < D / 16; ++i) acc[i] = f32x4{0.f, 0.f, 0.f, 0.f};

  // Key tiles are fetched in order through running pointers; a full tile
  // uses offsets computed once, a ragged one clamps (stage_load).
  Stage<T, D> stK, stV;
  frag pn[2];
  const StageOff<T, D> soK = stage_offsets<T, D>(a.k.st), soV = stage_offsets<T, D>(a.v.st);
  const T* Kn = K + (int64_t)cr.t0 * kBlk * a.k.st;
  const T* Vn = V + (int64_t)cr.t0 * kBlk * a.v.st;
  const T* Pn = LOADP ? Pm + cr.t0 * kBlk + stream_index(0, g, 0) : nullptr;
  auto fetch = [&](int nb) __attribute__((always_inline)) {
    const int n1 = nb * kBlk;
    if constexpr (!LOADP) {
      // Recompute: tile-indexed clamped loads, measured faster for this
      // variant than the running-pointer form below.
      stage_load<T, D>(stK, K + (int64_t)n1 * a.k.st, a.k.st, T_ - n1, D);
      stage_load<T, D>(stV, V + (int64_t)n1 * a.v.st, a.v.st, T_ - n1, D);
      return;
    }
    if (n1 + kBlk <= T_) {
      stage_load_full<T, D>(stK, Kn, soK);
      stage_load_full<T, D>(stV, Vn, soV);
      if constexpr (LOADP) {
        pn[0] = load_frag_g<T>(Pn);
        pn[1] = load_frag_g<T>(Pn + 32);
      }
    } else {
      stage_load<T, D>(stK, Kn, a.k.st, T_ - n1, D);
      stage_load<T, D>(stV, Vn, a.v.st, T_ - n1, D);
      if constexpr (LOADP) load_p_frags<T>(pn, Pm, n1, T_);
    }
    Kn += kBlk * a.k.st;
    Vn += kBlk * a.v.st;
    if constexpr (LOADP) Pn += kBlk;
  };
  // Direct loads of key tile nb into buffer set `par` (kDma).
  const TileDma<T, D> dd;
  int oK[TileDma<T, D>::kPerWave], oV[TileDma<T, D>::kPerWave];
  if constexpr (kDma) {
    dd.offsets(oK, a.k.st);
    dd.offsets(oV, a.v.st);
  }
  auto fetch_dma = [&](int nb, auto par) __attribute__((always_inline)) {
    const int n1 = nb * kBlk;
    if (n1 + kBlk <= T_) {
      dd.load_full(set_k(par), Kn, oK);
      dd.load_full(set_v(par), Vn, oV);
      if constexpr (LOADP) {
        pn[0] = load_frag_g<T>(Pn);
        pn[1] = load_frag_g<T>(Pn + 32);
      }
    } else {
      dd.load_ragged(set_k(par), Kn, a.k.st, T_ - n1, D);
      dd.load_ragged(set_v(par), Vn, a.v.st, T_ - n1, D);
      if constexpr (LOADP) load_p_frags<T>(pn, Pm, n1, T_);
      dma_wait();
    }
    Kn += kBlk * a.k.st;
    Vn += kBlk * a.v.st;
    if constexpr (LOADP) Pn += kBlk;
  };
  if constexpr (kPar)
    fetch_dma(cr.t0, Parity<0>{});
  else if constexpr (kRt)
    fetch_dma(cr.t0, RtBuf{0});
  else
    fetch(cr.t0);
  // Tile nb from buffer set `par`; `prefetch`: 1 fetch tile nb + 1, 2 fetch it
  // if it exists, 0 none.
  auto tile = [&](int nb, auto prefetch, auto par) __attribute__((always_inline)) {
    const int n0 = nb * kBlk;
    if constexpr (kDma) {
      dma_wait();       // this wave's loads of tile nb
      __syncthreads();  // everyone's, and everyone is done with the other set
    } else {
      __syncthreads();
      stage_store_rows<T, D>(stK, sK0);
      stage_store_rows<T, D>(stV, sV0);
      __syncthreads();
    }
    const T* cK = set_k(par);
    const T* cV = set_v(par);
    Tile p;
    if constexpr (LOADP) frags_to_tile<T>(p, pn);
    if constexpr (kDma) {
      if constexpr (decltype(prefetch)::value == 1) fetch_dma(nb + 1, other_buf(par));
      if constexpr (decltype(prefetch)::value == 2)
        if (nb + 1 < cr.t1) fetch_dma(nb + 1, other_buf(par));
    } else {
      if constexpr (decltype(prefetch)::value == 1) fetch(nb + 1);
      if constexpr (decltype(prefetch)::value == 2)
        if (nb + 1 < cr.t1) fetch(nb + 1);
    }
    if constexpr (!LOADP) {
      p.zero();
      mm_d<T, D>(p, cK, qf);
      recompute_p_row<T, XM>(p, a, brow, n0, lse2, a.scale_log2);
    }
    if (mk.tile(nb)) {
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int j = 0; j < 8; ++j)
          p.set(kb, j, mk.masked(n0 + stream_index(kb, g, j)) ? 0.f : p.at(kb, j));
    }
    Tile dp;
#pragma unroll
    for (int q4 = 0; q4 < 4; ++q4) dp.q[q4] = mDm4;
    mm_d<T, D>(dp, cV, dof);  // dP - D
    frag dsf[2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      float v[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) v[j] = p.at(kb, j) * dp.at(kb, j);
      dsf[kb] = vals_frag<T>(v);
    }
    mm_s<T, D>(acc, cK, dsf);
  };
  if constexpr (kPar && D == 64) {
    // Pairs of tiles with unconditional prefetch; the last one or two peeled.
    int nb = cr.t0;
    for (; nb + 2 < cr.t1; nb += 2) {
      tile(nb, Parity<1>{}, Parity<0>{});
      tile(nb + 1, Parity<1>{}, Parity<1>{});
    }
    if (nb + 1 < cr.t1) {
      tile(nb, Parity<1>{}, Parity<0>{});
      tile(nb + 1, Parity<0>{}, Parity<1>{});
    } else {
      tile(nb, Parity<0>{}, Parity<0>{});
    }
  } else if constexpr (kPar) {
    for (int nb = cr.t0; nb < cr.t1; nb += 2) {
      tile(nb, Parity<2>{}, Parity<0>{});
      if (nb + 1 < cr.t1) tile(nb + 1, Parity<2>{}, Parity<1>{});
    }
  } else if constexpr (kRt) {
    // The last tile is peeled off the loop, so inside it the next tile's
    // fetch is unconditional and its registers need no copies across
    // iterations.
    for (int nb = cr.t0; nb + 1 < cr.t1; ++nb) tile(nb, Parity<1>{}, RtBuf{(nb - cr.t0) & 1});
    tile(cr.t1 - 1, Parity<0>{}, RtBuf{(cr.t1 - 1 - cr.t0) & 1});
  } else if constexpr (LOADP) {
    for (int nb = cr.t0; nb + 1 < cr.t1; ++nb) tile(nb, Parity<1>{}, Parity<0>{});
    tile(cr.t1 - 1, Parity<0>{}, Parity<0>{});
  } else {
    for (int nb = cr.t0; nb < cr.t1; ++nb) tile(nb, Parity<2>{}, Parity<0>{});
  }
  if (cr.nch == 1)
    store_acc_rows<T, D>(at<T>(a.dq, b, h), a.dq.st, m, T_, acc, a.scale);
  else
    store_acc_partial<D>(a.ws_acc + part_index(a, bh, nblk, mb, ch) * kBlk * D, rl, acc);
}

// ---------------------------------------------------------------------------
// Waves per SIMD the dK/dV kernel is compiled for: recompute at D = 64 caps
// registers for VGPR accumulators; the saved-P 16-bit kernels (direct loads)
// for three waves at D = 64 and two at D = 128.
template <typename T, int D, bool LOADP, bool DV_ONLY>
struct DkdvWaves {
  static constexpr bool kDma = LOADP && !DV_ONLY && sizeof(T) == 2;
  static constexpr int value = kDma ? (D == 64 ? 3 : 2) : AccWaves<!LOADP && D == 64>::value;
};

template <typename T, int D, bool LOADP, bool DV_ONLY, bool XM>
__global__ __launch_bounds__(kThreads)
__attribute__((amdgpu_waves_per_eu(DkdvWaves<T, D, LOADP, DV_ONLY>::value))) void k_bwd_dkdv(Params a, Params dqc,
                                                                                              int nx) {
  typedef Elem<T> E;
  typedef typename E::frag frag;
  typedef Lds<T, D> L;
  typedef Lds<T, kBlk> LP;
  constexpr bool kNeedQ = !DV_ONLY || !LOADP;
  // Staged row statistics of the streamed tile: D (unless DV_ONLY), then lse
  // (recompute only).
  constexpr int kNS = (DV_ONLY ? 0 : 1) + (LOADP ? 0 : 1);
  constexpr int kSD = 0, kSL = DV_ONLY ? 0 : 1;
  // Saved-P 16-bit D = 64 tiles (dO, Q, P and the rowsum slice) stream
  // straight into two LDS buffer sets (TileDma) in distinct arrays with a
  // compile-time role per loop step, so that the current tile's LDS reads
  // need not wait for the next tile's loads.
  // At D = 128 (kMix) P stays staged through registers into one buffer: two
  // sets of all three tiles would need 80 KB of LDS, one workgroup per CU.
  constexpr bool kDma = !DV_ONLY && L::kSwizzle && (LOADP || D == 64);
  constexpr bool kMix = kDma && D == 128;
  // The next tile's loads are issued after this tile's P reads: issued before
  // them, the compiler waits for the outstanding direct loads before one of
  // those transposed reads.
  constexpr bool kLateFetch = kDma && LOADP;
  constexpr int kQE = kNeedQ ? L::kRowElems : 8, kPE = LOADP ? LP::kRowElems : 8, kSE = kNS > 0 ? kNS * kBlk : 4;
  __shared__ __align__(16) T sdO0[L::kRowElems];
  __shared__ __align__(16) T sQ0[kQE];
  __shared__ __align__(16) T sP0[kPE];
  __shared__ __align__(16) float sS0[kSE];
  __shared__ __align__(16) T sdO1[kDma ? L::kRowElems : 8];
  __shared__ __align__(16) T sQ1[kDma ? kQE : 8];
  __shared__ __align__(16) T sP1[kDma && !kMix ? kPE : 8];
  __shared__ __align__(16) float sS1[kDma ? kSE : 4];
  struct Bufs {
    T *dout, *q, *p;
    float* st;
  };
  auto bufs = [&](auto par) __attribute__((always_inline)) -> Bufs {
    if constexpr (decltype(par)::value == 0)
      return Bufs{sdO0, sQ0, sP0, sS0};
    else
      return Bufs{sdO1, sQ1, kMix ? sP0 : sP1, sS1};
  };

  const int T_ = a.T;
  const int nblk = (T_ + kBlk - 1) / kBlk;
  const Slot sl = grid_slot();
  // Workgroups past the first nx columns of the grid finish the preceding dQ
  // launch's split blocks (its partials are complete in stream order), in the
  // tail of this launch rather than in a launch of their own.
  if (sl.x >= nx) {
    combine_sum_block<T, D>(dqc, kOutDQ, sl.x - nx, sl.y);
    return;
  }
  const Item it = launch_item<XM>(a, sl.x, nblk);  // causal: column 0 has the most tiles
  if (it.blk < 0) return;
  const int nb = it.blk, ch = it.ch;
  const int bh = sl.y, b = bh / a.H, h = bh % a.H;
  const Range rg = col_block_range(nb, nblk, T_, a.causal, XM ? a.win : 0, a.win_kind);
  const Chunk cr = chunk_of(rg.lo, rg.hi, ch, a.chunk);
  if (ch >= cr.nch) return;
  const int n0 = nb * kBlk;
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63, c = lane & 15, g = lane >> 4;
  const int cl = 16 * w + c;
  const int n = n0 + cl;
  const ColMask<XM> mk(a, nb, n);
  const T* bcol = (XM && !LOADP && a.bias.p) ? at<const T>(a.bias, b, h) + (n < T_ ? n : 0) : nullptr;

  const T* Q = at<const T>(a.q, b, h);
  const T* K = at<const T>(a.k, b, h);
  const T* V = at<const T>(a.v, b, h);
  const T* dO = at<const T>(a.dout, b, h);
  const T* Pb = LOADP ? at<const T>(a.p, b, h) : nullptr;
  const float* rs = DV_ONLY ? nullptr : a.rowsum_in + (int64_t)bh * T_;
  const float* lse = LOADP ? nullptr : a.lse + (int64_t)bh * T_;

  frag vf[D / 32], kf[D / 32];
#pragma unroll
  for (int ks = 0; ks < D / 32; ++ks) {
    // negated: dP's MFMAs start from the streamed rows' D and give D - dP;
    // kept as computed (left to itself the compiler redoes the negation per tile)
    if constexpr (!DV_ONLY) {
      vf[ks] = scale_frag<T>(load_frag_row<T>(V, a.v.st, n, T_, 32 * ks + 8 * g), -1.f);
      asm volatile("" : "+v"(vf[ks]));
    }
    if constexpr (!LOADP) kf[ks] = load_frag_row<T>(K, a.k.st, n, T_, 32 * ks + 8 * g);
  }

  f32x4 acc_dv[D / 16], acc_dk[D / 16];
#pragma unroll
  for (int i = 0; i < D / 16; ++i) acc_dv[i] = acc_dk[i] = f32x4{0.f, 0.f, 0.f, 0.f};

  // Query tiles are fetched in order through running pointers with clamped
  // addressing (stage_load).
  Stage<T, D> stdO, stQ;
  Stage<T, kBlk> stP;
  float stv = 0.f;
  const int64_t t0r = (int64_t)cr.t0 * kBlk;
  const T* dOn = dO + t0r * a.dout.st;
  const T* Qn = Q + t0r * a.q.st;
  const T* Pn = LOADP ? Pb + t0r * a.p.st + n0 : nullptr;
  const bool cols_full = n0 + kBlk <= T_;
  auto load_tile = [&](int mb) __attribute__((always_inline)) {
    const int m0 = mb * kBlk;
    stage_load<T, D>(stdO, dOn, a.dout.st, T_ - m0, D);
    if constexpr (kNeedQ) stage_load<T, D>(stQ, Qn, a.q.st, T_ - m0, D);
    if constexpr (LOADP) stage_load<T, kBlk>(stP, Pn, a.p.st, T_ - m0, T_ - n0);
    if constexpr (kNS > 0) stv = stat_load<kNS>(DV_ONLY ? lse : rs, lse, nullptr, nullptr, m0, T_ - m0);
    dOn += kBlk * a.dout.st;
    if constexpr (kNeedQ) Qn += kBlk * a.q.st;
    if constexpr (LOADP) Pn += kBlk * a.p.st;
  };
  // Direct loads of query tile mb into buffer set `par` (kDma), in order
  // through the same running pointers.
  const TileDma<T, D> dd;
  const TileDma<T, kBlk> dpt;
  int odO[TileDma<T, D>::kPerWave], oQ[TileDma<T, D>::kPerWave], oP[TileDma<T, kBlk>::kPerWave];
  if constexpr (kDma) {
    dd.offsets(odO, a.dout.st);
    dd.offsets(oQ, a.q.st);
    if constexpr (LOADP) dpt.offsets(oP, a.p.st);
  }
  const StatDma<kNS> sdma(DV_ONLY ? lse : rs, lse, nullptr, nullptr);
  auto dma_tile = [&](int mb, auto par) __attribute__((always_inline)) {
    const int m0 = mb * kBlk;
    const Bufs bf = bufs(par);
    if (m0 + kBlk <= T_ && cols_full) {
      dd.load_full(bf.dout, dOn, odO);
      dd.load_full(bf.q, Qn, oQ);
      if constexpr (LOADP && !kMix) dpt.load_full(bf.p, Pn, oP);
    } else {
      dd.load_ragged(bf.dout, dOn, a.dout.st, T_ - m0, D);
      dd.load_ragged(bf.q, Qn, a.q.st, T_ - m0, D);
      if constexpr (LOADP && !kMix) dpt.load_ragged(bf.p, Pn, a.p.st, T_ - m0, T_ - n0);
      dma_wait();
    }
    sdma.load(bf.st, m0, T_ - m0);
    if constexpr (kMix) stage_load<T, kBlk>(stP, Pn, a.p.st, T_ - m0, T_ - n0);
    dOn += kBlk * a.dout.st;
    Qn += kBlk * a.q.st;
    if constexpr (LOADP) Pn += kBlk * a.p.st;
  };
  if constexpr (kDma)
    dma_tile(cr.t0, Parity<0>{});
  else
    load_tile(cr.t0);
  // Tile mb from buffer set `par`; `prefetch`: 1 fetch tile mb + 1, 2 fetch it
  // if it exists, 0 none.
  auto tile = [&](int mb, auto prefetch, auto par) __attribute__((always_inline)) {
    const int m0 = mb * kBlk;
    constexpr int P = decltype(par)::value;
    if constexpr (kDma) {
      dma_wait();       // this wave's loads of tile mb
      __syncthreads();  // everyone's; everyone is also done with the other set
      if constexpr (kMix) {
        stage_store_rows<T, kBlk>(stP, sP0);
        __syncthreads();
      }
      if constexpr (!kLateFetch) {
        if constexpr (decltype(prefetch)::value == 1) dma_tile(mb + 1, Parity<1 - P>{});
        if constexpr (decltype(prefetch)::value == 2)
          if (mb + 1 < cr.t1) dma_tile(mb + 1, Parity<1 - P>{});
      }
    } else {
      __syncthreads();
      stage_store_rows<T, D>(stdO, sdO0);
      if constexpr (kNeedQ) stage_store_rows<T, D>(stQ, sQ0);
      if constexpr (LOADP) stage_store_rows<T, kBlk>(stP, sP0);
      if constexpr (kNS > 0) stat_store<kNS>(stv, sS0);
      __syncthreads();
      if constexpr (decltype(prefetch)::value == 1) load_tile(mb + 1);
      if constexpr (decltype(prefetch)::value == 2)
        if (mb + 1 < cr.t1) load_tile(mb + 1);
    }
    const Bufs cb = bufs(par);
    const T* cdO = cb.dout;
    const T* cQ = cb.q;
    const T* cP = cb.p;
    const float* cS = cb.st;

    // P(m, n) for streamed m = m0 + 32kb + 8g + j, stationary n.
    Tile p;
    if constexpr (LOADP) {
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        const frag f = load_frag_tr<T, kBlk>(cP, 32 * kb, 16 * w);
#pragma unroll
        for (int j = 0; j < 8; ++j) p.set(kb, j, E::f32(f[j]));
      }
      if constexpr (kLateFetch) {
        if constexpr (decltype(prefetch)::value == 1) dma_tile(mb + 1, Parity<1 - P>{});
        if constexpr (decltype(prefetch)::value == 2)
          if (mb + 1 < cr.t1) dma_tile(mb + 1, Parity<1 - P>{});
      }
    } else {
      p.zero();
      mm_d<T, D>(p, cQ, kf);
      recompute_p_col<T, XM>(p, a, bcol, m0, cS, kSL, a.scale_log2);
    }
    if (mk.tile(mb)) {
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int j = 0; j < 8; ++j)
          p.set(kb, j, mk.masked(m0 + stream_index(kb, g, j)) ? 0.f : p.at(kb, j));
    }
    frag pf[2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) pf[kb] = tile_frag<T>(p, kb);
    mm_s<T, D>(acc_dv, cdO, pf);
    if constexpr (!DV_ONLY) {
      Tile dp;
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        float d8[8];
        stat_read8(d8, cS, kSD, kb);
        dp.q[2 * kb] = f32x4{d8[0], d8[1], d8[2], d8[3]};
        dp.q[2 * kb + 1] = f32x4{d8[4], d8[5], d8[6], d8[7]};
      }
      mm_d<T, D>(dp, cdO, vf);  // D - dP
      frag dsf[2];
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        float v[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = p.at(kb, j) * dp.at(kb, j);  // -dS
        dsf[kb] = vals_frag<T>(v);
      }
      mm_s<T, D>(acc_dk, cQ, dsf);  // -dK / s
    }
  };
  if constexpr (kDma) {
    for (int mb = cr.t0; mb < cr.t1; mb += 2) {
      tile(mb, Parity<2>{}, Parity<0>{});
      if (mb + 1 < cr.t1) tile(mb + 1, Parity<2>{}, Parity<1>{});
    }
  } else {
    for (int mb = cr.t0; mb < cr.t1; ++mb) tile(mb, Parity<2>{}, Parity<0>{});
  }
  if (cr.nch == 1) {
    store_acc_rows<T, D>(at<T>(a.dv, b, h), a.dv.st, n, T_, acc_dv, 1.f);
    if constexpr (!DV_ONLY) store_acc_rows<T, D>(at<T>(a.dk, b, h), a.dk.st, n, T_, acc_dk, -a.scale);
  } else {
    float* base = a.ws_acc + part_index(a, bh, nblk, nb, ch) * 2 * kBlk * D;
    store_acc_partial<D>(base, cl, acc_dv);
    if constexpr (!DV_ONLY) {
#pragma unroll
      for (int i = 0; i < D / 16; ++i) acc_dk[i] = -acc_dk[i];
      store_acc_partial<D>(base + kBlk * D, cl, acc_dk);
    }
  }
}

// ---------------------------------------------------------------------------
// rowsum[m] = sum_n P[m,n] * (dO*V^T)[m,n]; causal skips tiles past the
// diagonal (they hold zeros in the math path).
template <typename T, int D, bool XM>
__global__ __launch_bounds__(kThreads) void k_bwd_rowsum(Params a) {
  typedef Elem<T> E;
  typedef typename E::frag frag;
  typedef Lds<T, D> L;
  __shared__ __align__(16) T sV[L::kRowElems];

  const int T_ = a.T;
  const Slot sl = grid_slot();
  const int bh = sl.y, b = bh / a.H, h = bh % a.H;
  const int nblk = (T_ + kBlk - 1) / kBlk;
  const int mb = a.causal ? (nblk - 1 - sl.x) : sl.x;
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63, c = lane & 15, g = lane >> 4;
  const int m = mb * kBlk + 16 * w + c;
  const bool row_ok = m < T_;
  const T* V = at<const T>(a.v, b, h);
  const T* dO = at<const T>(a.dout, b, h);
  const T* Pm = at<const T>(a.p, b, h) + (int64_t)(row_ok ? m : 0) * a.p.st;

  frag dof[D / 32];
#pragma unroll
  for (int ks = 0; ks < D / 32; ++ks) dof[ks] = load_frag_row<T>(dO, a.dout.st, m, T_, 32 * ks + 8 * g);

  float sum = 0.f;
  const Range rg = row_block_range(mb, nblk, T_, a.causal, XM ? a.win : 0, a.win_kind);
  const RowMask<XM> mk(a, mb, m);
  Stage<T, D> stV;
  stage_load<T, D>(stV, V + (int64_t)rg.lo * kBlk * a.v.st, a.v.st, T_ - rg.lo * kBlk, D);
  for (int nb = rg.lo; nb < rg.hi; ++nb) {
    const int n0 = nb * kBlk;
    __syncthreads();
    stage_store_rows<T, D>(stV, sV);
    __syncthreads();
    if (nb + 1 < rg.hi) stage_load<T, D>(stV, V + (int64_t)(n0 + kBlk) * a.v.st, a.v.st, T_ - n0 - kBlk, D);
    frag pr[2];
    load_p_frags<T>(pr, Pm, n0, T_);
    Tile p, dp;
    frags_to_tile<T>(p, pr);
    if (mk.tile(nb)) {
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int j = 0; j < 8; ++j)
          p.set(kb, j, mk.masked(n0 + stream_index(kb, g, j)) ? 0.f : p.at(kb, j));
    }
    dp.zero();
    mm_d<T, D>(dp, sV, dof);
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int j = 0; j < 8; ++j) sum += p.at(kb, j) * dp.at(kb, j);
  }
  sum = group_sum(sum);
  if (row_ok && g == 0) a.rowsum_out[(int64_t)bh * T_ + m] = sum;
}

// ---------------------------------------------------------------------------
template <typename T, int D, bool XM>
static void launch_dq_x(const Params& a, bool load_p, dim3 grid, hipStream_t st) {
  const TimedLaunch tl(st, kTagDq);
  if (load_p)
    hipLaunchKernelGGL((k_bwd_dq<T, D, true, XM>), grid, dim3(kThreads), 0, st, a);
  else
    hipLaunchKernelGGL((k_bwd_dq<T, D, false, XM>), grid, dim3(kThreads), 0, st, a);
}

template <typename T, int D>
static hipError_t launch_dq_t(int dtype, const Params& a, bool load_p, hipStream_t st, bool combine) {
  const int nblk = (a.T + kBlk - 1) / kBlk;
  dim3 grid(nblk * a.nchunk_max, a.B * a.H);
  if (extended_mask(a))
    launch_dq_x<T, D, true>(a, load_p, grid, st);
  else
    launch_dq_x<T, D, false>(a, load_p, grid, st);
  if (combine && a.nchunk_max > 1) return launch_combine_sum(dtype, D, a, kOutDQ, st);
  return hipGetLastError();
}

template <typename T, int D, bool XM>
static void launch_dkdv_x(const Params& a, bool load_p, bool dv_only, dim3 grid, hipStream_t st, const Params& c,
                          int nx) {
  const TimedLaunch tl(st, kTagDkdv);
  if (load_p) {
    if (dv_only)
      hipLaunchKernelGGL((k_bwd_dkdv<T, D, true, true, XM>), grid, dim3(kThreads), 0, st, a, c, nx);
    else
      hipLaunchKernelGGL((k_bwd_dkdv<T, D, true, false, XM>), grid, dim3(kThreads), 0, st, a, c, nx);
  } else {
    if (dv_only)
      hipLaunchKernelGGL((k_bwd_dkdv<T, D, false, true, XM>), grid, dim3(kThreads), 0, st, a, c, nx);
    else
      hipLaunchKernelGGL((k_bwd_dkdv<T, D, false, false, XM>), grid, dim3(kThreads), 0, st, a, c, nx);
  }
}

template <typename T, int D>
static hipError_t launch_dkdv_t(int dtype, const Params& a, bool load_p, bool dv_only, hipStream_t st,
                                const Params* dqc) {
  const int nblk = (a.T + kBlk - 1) / kBlk;
  const int nx = nblk * a.nchunk_max;
  const bool fold = dqc && dqc->nchunk_max > 1;
  dim3 grid(nx + (fold ? nblk * CombineSlot<D>::kSub : 0), a.B * a.H);
  const Params& c = fold ? *dqc : a;
  if (extended_mask(a))
    launch_dkdv_x<T, D, true>(a, load_p, dv_only, grid, st, c, nx);
  else
    launch_dkdv_x<T, D, false>(a, load_p, dv_only, grid, st, c, nx);
  if (a.nchunk_max > 1) return launch_combine_sum(dtype, D, a, dv_only ? kOutDV : kOutDKDV, st);
  return hipGetLastError();
}

template <typename T, int D>
static hipError_t launch_rowsum_t(const Params& a, hipStream_t st) {
  dim3 grid((a.T + kBlk - 1) / kBlk, a.B * a.H);
  if (extended_mask(a))
    hipLaunchKernelGGL((k_bwd_rowsum<T, D, true>), grid, dim3(kThreads), 0, st, a);
  else
    hipLaunchKernelGGL((k_bwd_rowsum<T, D, false>), grid, dim3(kThreads), 0, st, a);
  return hipGetLastError();
}

template <typename T, int D, bool XM>
static int occupancy_dq_t(bool load_p) {
  return load_p ? occupancy_of(k_bwd_dq<T, D, true, XM>) : occupancy_of(k_bwd_dq<T, D, false, XM>);
}

template <typename T, int D, bool XM>
static int occupancy_dkdv_t(bool load_p) {
  return load_p ? occupancy_of(k_bwd_dkdv<T, D, true, false, XM>)
                : occupancy_of(k_bwd_dkdv<T, D, false, false, XM>);
}

int occupancy_dq(int dtype, int D, bool load_p, bool xm) {
  if (xm) DISPATCH_DTYPE_D(dtype, D, return occupancy_dq_t<ElemT, kD, true>(load_p));
  else DISPATCH_DTYPE_D(dtype, D, return occupancy_dq_t<ElemT, kD, false>(load_p));
  return 0;
}

int occupancy_dkdv(int dtype, int D, bool load_p, bool xm) {
  if (xm) DISPATCH_DTYPE_D(dtype, D, return occupancy_dkdv_t<ElemT, kD, true>(load_p));
  else DISPATCH_DTYPE_D(dtype, D, return occupancy_dkdv_t<ElemT, kD, false>(load_p));
  return 0;
}

hipError_t launch_bwd_dq(int dtype, int D, const Params& a, bool load_p, hipStream_t st, bool combine) {
  DISPATCH_DTYPE_D(dtype, D, return launch_dq_t<ElemT, kD>(dtype, a, load_p, st, combine));
  return hipErrorInvalidValue;
}

hipError_t launch_bwd_dkdv(int dtype, int D, const Params& a, bool load_p, bool dv_only, hipStream_t st,
                           const Params* dq_combine) {
  DISPATCH_DTYPE_D(dtype, D, return launch_dkdv_t<ElemT, kD>(dtype, a, load_p, dv_only, st, dq_combine));
  return hipErrorInvalidValue;
}

hipError_t launch_bwd_rowsum(int dtype, int D, const Params& a, hipStream_t st) {
  DISPATCH_DTYPE_D(dtype, D, return launch_rowsum_t<ElemT, kD>(a, st));
  return hipErrorInvalidValue;
}

}  // namespace ttt
