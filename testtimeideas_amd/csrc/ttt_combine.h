// ttt_combine.h — device helpers of the combine step (ttt_combine.hip): the
// workgroup layout of a combine launch, chunk counts, in-order sums of fp32
// partials, and the plain-sum combine of one workgroup, which ttt_bwd.hip
// also runs inside the dK/dV launch for the dQ partials.
//
// Each main-kernel workgroup of a split block wrote fp32 partials to the
// workspace: accumulators [part][nacc] as 64 x D blocks in part_off layout
// (ttt_common.h) and row scalars [part][nsc][64], part = (bh*nblk + block)*
// nchunk_max + chunk.  The combine reads every chunk of a block in chunk
// order (so results do not depend on scheduling).  A block's 64 x D outputs
// are covered by D/16 workgroups; thread t of workgroup `sub` owns the 4-wide
// slot s = 256*sub + t (CombineSlot).
#pragma once
#include "ttt_common.h"
#include "ttt_launch.h"

namespace ttt {

// Slot s of a block is the 16-byte run at 4*s floats of its part_off layout:
// consecutive threads read consecutive runs, and each wave's 16 rows x 16
// columns are written to the output together.
template <int D>
struct CombineSlot {
  static constexpr int kSub = kBlk * (D / 4) / kThreads;  // workgroups per block
  int blk, r, d0;
  __device__ __forceinline__ explicit CombineSlot(int bx) {
    blk = bx / kSub;
    const int s = (bx % kSub) * kThreads + threadIdx.x;
    const int q = s % (4 * D);
    r = 16 * (s / (4 * D)) + ((q >> 2) & 15);
    d0 = 16 * (q >> 6) + 4 * (q & 3);
  }
};

__device__ __forceinline__ int block_nch(const Params& a, int blk, int nblk, bool col) {
  const Range r = col ? col_block_range(blk, nblk, a.T, a.causal, a.win, a.win_kind)
                      : row_block_range(blk, nblk, a.T, a.causal, a.win, a.win_kind);
  return (r.hi - r.lo + a.chunk - 1) / a.chunk;
}

// Chunks whose loads a thread issues together before adding them.  The
// loads of a batch are unconditional (chunk indices past nch-1 repeat the
// last chunk) so that none waits for another; the adds still run in chunk
// order 0, 1, ..., nch-1.
constexpr int kBatch = 8;

// out[i] = sum over chunks k (in order) of accumulator a0 + i at (r, d0..d0+3).
template <int D, int NA>
__device__ __forceinline__ void sum_parts(f32x4* out, const float* ws, int64_t p0, int nch, int nacc, int a0,
                                          int r, int d0) {
#pragma unroll
  for (int i = 0; i < NA; ++i) out[i] = f32x4{0.f, 0.f, 0.f, 0.f};
  const float* base = ws + (p0 * nacc + a0) * kBlk * D + part_off<D>(r, d0);
  const int64_t step = (int64_t)nacc * kBlk * D;
  for (int k0 = 0; k0 < nch; k0 += kBatch) {
    f32x4 x[kBatch][NA];
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      const int k = min(k0 + u, nch - 1);
#pragma unroll
      for (int i = 0; i < NA; ++i) x[u][i] = *reinterpret_cast<const f32x4*>(base + k * step + i * kBlk * D);
    }
#pragma unroll
    for (int u = 0; u < kBatch; ++u)
      if (k0 + u < nch) {
#pragma unroll
        for (int i = 0; i < NA; ++i) out[i] += x[u][i];
      }
  }
}

// s[j] = sum over chunks k (in order) of row scalar j (of NS) at row r.
template <int NS>
__device__ __forceinline__ void sum_scalars(float* s, const float* ws_sc, int64_t p0, int nch, int r) {
#pragma unroll
  for (int j = 0; j < NS; ++j) s[j] = 0.f;
  for (int k0 = 0; k0 < nch; k0 += kBatch) {
    float x[kBatch][NS];
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      const int k = min(k0 + u, nch - 1);
#pragma unroll
      for (int j = 0; j < NS; ++j) x[u][j] = ws_sc[(p0 + k) * NS * kBlk + j * kBlk + r];
    }
#pragma unroll
    for (int u = 0; u < kBatch; ++u)
      if (k0 + u < nch) {
#pragma unroll
        for (int j = 0; j < NS; ++j) s[j] += x[u][j];
      }
  }
}

template <typename T>
__device__ __forceinline__ void store_slot(const View& o, int b, int h, int row, int d0, f32x4 v) {
  store4<T>(at<T>(o, b, h) + (int64_t)row * o.st + d0, v);
}

// ---------------------------------------------------------------------------
// Plain sums (O of the save_p forward, dQ, dK/dV, GK/GV) for combine
// workgroup (bx, by) of a grid of nblk * CombineSlot<D>::kSub by B*H.
template <typename T, int D>
__device__ __forceinline__ void combine_sum_block(const Params& a, int which, int bx, int by) {
  const int T_ = a.T;
  const int nblk = (T_ + kBlk - 1) / kBlk;
  const CombineSlot<D> cs(bx);
  const int bh = by, b = bh / a.H, h = bh % a.H;
  const bool col = which == kOutDKDV || which == kOutDV || which == kOutGKGV;
  const int nch = block_nch(a, cs.blk, nblk, col);
  if (nch <= 1) return;
  const int row = cs.blk * kBlk + cs.r;
  if (row >= T_) return;
  const int64_t p0 = part_index(a, bh, nblk, cs.blk, 0);
  if (which == kOutO || which == kOutDQ) {
    f32x4 v;
    sum_parts<D, 1>(&v, a.ws_acc, p0, nch, 1, 0, cs.r, cs.d0);
    if (which == kOutO)
      store_slot<T>(a.o, b, h, row, cs.d0, v);
    else
      store_slot<T>(a.dq, b, h, row, cs.d0, v * a.scale);
    return;
  }
  // two-accumulator column kernels: index 0 = dV / GK, index 1 = dK / GV
  const bool gg = which == kOutGKGV;
  if (which == kOutDV) {
    f32x4 v;
    sum_parts<D, 1>(&v, a.ws_acc, p0, nch, 2, 0, cs.r, cs.d0);
    store_slot<T>(a.dv, b, h, row, cs.d0, v);
    return;
  }
  f32x4 v[2];
  sum_parts<D, 2>(v, a.ws_acc, p0, nch, 2, 0, cs.r, cs.d0);
  store_slot<T>(gg ? a.gk_out : a.dv, b, h, row, cs.d0, v[0] * (gg ? a.scale : 1.f));
  store_slot<T>(gg ? a.gv_out : a.dk, b, h, row, cs.d0, v[1] * (gg ? 1.f : a.scale));
}

// ---------------------------------------------------------------------------
// Grad-grad row pass, combine workgroup (bx, by): E and F from the chunk
// sums (written when write_ef), then GQ (and GdO).
// Accumulators: 0..2 = dS*gK + Z1*K, Z2*K, P*K; 3..4 = P*gV + (P o gdS)*V, P*V.
// Scalars: 0 = E, 1 = rowsum(Z1), 2 = rowsum(Z2).
// The dQ form (a.dq.p set, no GdO): accumulators 0..1 = dS*gK + Z1*K, P*K;
// scalar 2 = X summed in fp32 (Xf); GQ = s*(acc0 - X acc1) - E dQ and
// F = Xf - E D.
template <typename T, int D, bool GDO>
__device__ __forceinline__ void combine_gg_row_block(const Params& a, int bx, int by, bool write_ef) {
  constexpr int NACC = GDO ? 5 : 3;
  const int T_ = a.T;
  const int nblk = (T_ + kBlk - 1) / kBlk;
  const CombineSlot<D> cs(bx);
  const int bh = by, b = bh / a.H, h = bh % a.H;
  const int nch = block_nch(a, cs.blk, nblk, false);
  if (nch <= 1) return;
  const int r = cs.r;
  const int row = cs.blk * kBlk + r;
  if (row >= T_) return;
  const int64_t p0 = part_index(a, bh, nblk, cs.blk, 0);
  if constexpr (!GDO) {
    if (a.dq.p) {
      float sc[3];
      sum_scalars<3>(sc, a.ws_sc, p0, nch, r);
      const float ev = sc[0], gv = sc[1];
      f32x4 t[2];
      sum_parts<D, 2>(t, a.ws_acc, p0, nch, 2, 0, r, cs.d0);
      const f32x4 dq = load4<T>(at<const T>(a.dq, b, h) + (int64_t)row * a.dq.st + cs.d0);
      store_slot<T>(a.gq_out, b, h, row, cs.d0, (t[0] - gv * t[1]) * a.scale - ev * dq);
      if (write_ef && cs.d0 == 0) {
        a.e[(int64_t)bh * T_ + row] = ev;
        a.f[(int64_t)bh * T_ + row] = sc[2] - ev * a.rowsum_in[(int64_t)bh * T_ + row];
      }
      return;
    }
  }
  float sc[3];
  sum_scalars<3>(sc, a.ws_sc, p0, nch, r);
  const float ev = sc[0], xv = sc[1], dv = sc[2];
  const float fv = xv - ev * dv;
  f32x4 t[3];
  sum_parts<D, 3>(t, a.ws_acc, p0, nch, NACC, 0, r, cs.d0);
  f32x4 acc = t[0];
  acc -= ev * t[1];
  acc = a.scale * (acc - fv * t[2]);
  store_slot<T>(a.gq_out, b, h, row, cs.d0, acc);
  if constexpr (GDO) {
    f32x4 u[2];
    sum_parts<D, 2>(u, a.ws_acc, p0, nch, NACC, 3, r, cs.d0);
    f32x4 go = u[0];
    go -= ev * u[1];
    store_slot<T>(a.gdout, b, h, row, cs.d0, go);
  }
  if (write_ef && cs.d0 == 0) {
    a.e[(int64_t)bh * T_ + row] = ev;
    a.f[(int64_t)bh * T_ + row] = fv;
  }
}

}  // namespace ttt
