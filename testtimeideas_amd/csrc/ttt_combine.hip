// ttt_combine.hip — finish blocks whose streamed loop was split into chunks.
//
// The combine kernels read every chunk's fp32 partials of a block in chunk
// order (layout and helpers in ttt_combine.h) and write the outputs.  Blocks
// with a single chunk were finished by the main kernel and are skipped here.
// A thread issues the loads of all accumulators of up to kBatch chunks
// together; the sums still run in chunk order.
#include "ttt_combine.h"

namespace ttt {

// ---------------------------------------------------------------------------
// Plain sums: O (save_p forward), dQ, dK/dV, GK/GV.
template <typename T, int D>
__global__ __launch_bounds__(kThreads) void k_combine_sum(Params a, int which) {
  combine_sum_block<T, D>(a, which, blockIdx.x, blockIdx.y);
}

// ---------------------------------------------------------------------------
// Online-softmax merge: partial (m_c, l_c, acc_c) in base-2 units.
template <typename T, int D>
__global__ __launch_bounds__(kThreads) void k_combine_fwd(Params a) {
  const int T_ = a.T;
  const int nblk = (T_ + kBlk - 1) / kBlk;
  const CombineSlot<D> cs(blockIdx.x);
  const int bh = blockIdx.y, b = bh / a.H, h = bh % a.H;
  const int nch = block_nch(a, cs.blk, nblk, false);
  if (nch <= 1) return;
  const int r = cs.r;
  const int row = cs.blk * kBlk + r;
  if (row >= T_) return;
  const int64_t p0 = part_index(a, bh, nblk, cs.blk, 0);
  float mm = -INFINITY;
  for (int k0 = 0; k0 < nch; k0 += kBatch) {
    float x[kBatch];
#pragma unroll
    for (int u = 0; u < kBatch; ++u) x[u] = a.ws_sc[(p0 + min(k0 + u, nch - 1)) * 2 * kBlk + r];
#pragma unroll
    for (int u = 0; u < kBatch; ++u) mm = fmaxf(mm, x[u]);  // repeats of the last chunk leave the max
  }
  float ll = 0.f;
  f32x4 v = f32x4{0.f, 0.f, 0.f, 0.f};
  for (int k0 = 0; k0 < nch; k0 += kBatch) {
    float mk[kBatch], lk[kBatch];
    f32x4 xk[kBatch];
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      const int64_t k = p0 + min(k0 + u, nch - 1);
      mk[u] = a.ws_sc[k * 2 * kBlk + r];
      lk[u] = a.ws_sc[k * 2 * kBlk + kBlk + r];
      xk[u] = *reinterpret_cast<const f32x4*>(a.ws_acc + k * kBlk * D + r * D + cs.d0);
    }
#pragma unroll
    for (int u = 0; u < kBatch; ++u)
      if (k0 + u < nch) {
        const float wk = fast_exp2(mk[u] - mm);
        ll += lk[u] * wk;
        v += wk * xk[u];
      }
  }
  store_slot<T>(a.o, b, h, row, cs.d0, v * (1.f / ll));
  if (cs.d0 == 0) a.lse[(int64_t)bh * T_ + row] = (mm + __log2f(ll)) * kLn2;
}

// ---------------------------------------------------------------------------
// Grad-grad row pass: E, F from chunk sums, then GQ (and GdO).
// Accumulators: 0..2 = dS*gK + Z1*K, Z2*K, P*K; 3..4 = P*gV + (P o gdS)*V, P*V.
// Scalars: 0 = E, 1 = rowsum(Z1), 2 = rowsum(Z2).
template <typename T, int D, bool GDO>
__global__ __launch_bounds__(kThreads) void k_combine_gg_row(Params a) {
  constexpr int NACC = GDO ? 5 : 3;
  const int T_ = a.T;
  const int nblk = (T_ + kBlk - 1) / kBlk;
  const CombineSlot<D> cs(blockIdx.x);
  const int bh = blockIdx.y, b = bh / a.H, h = bh % a.H;
  const int nch = block_nch(a, cs.blk, nblk, false);
  if (nch <= 1) return;
  const int r = cs.r;
  const int row = cs.blk * kBlk + r;
  if (row >= T_) return;
  const int64_t p0 = part_index(a, bh, nblk, cs.blk, 0);
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
  if (cs.d0 == 0) {
    a.e[(int64_t)bh * T_ + row] = ev;
    a.f[(int64_t)bh * T_ + row] = fv;
  }
}

// ---------------------------------------------------------------------------
template <typename T, int D>
static hipError_t combine_sum_t(const Params& a, int which, hipStream_t st) {
  dim3 grid((a.T + kBlk - 1) / kBlk * CombineSlot<D>::kSub, a.B * a.H);
  hipLaunchKernelGGL((k_combine_sum<T, D>), grid, dim3(kThreads), 0, st, a, which);
  return hipGetLastError();
}

template <typename T, int D>
static hipError_t combine_fwd_t(const Params& a, hipStream_t st) {
  dim3 grid((a.T + kBlk - 1) / kBlk * CombineSlot<D>::kSub, a.B * a.H);
  hipLaunchKernelGGL((k_combine_fwd<T, D>), grid, dim3(kThreads), 0, st, a);
  return hipGetLastError();
}

template <typename T, int D>
static hipError_t combine_gg_row_t(const Params& a, bool gdo, hipStream_t st) {
  dim3 grid((a.T + kBlk - 1) / kBlk * CombineSlot<D>::kSub, a.B * a.H);
  if (gdo)
    hipLaunchKernelGGL((k_combine_gg_row<T, D, true>), grid, dim3(kThreads), 0, st, a);
  else
    hipLaunchKernelGGL((k_combine_gg_row<T, D, false>), grid, dim3(kThreads), 0, st, a);
  return hipGetLastError();
}

hipError_t launch_combine_sum(int dtype, int D, const Params& a, int which, hipStream_t st) {
  DISPATCH_DTYPE_D(dtype, D, return combine_sum_t<ElemT, kD>(a, which, st));
  return hipErrorInvalidValue;
}

hipError_t launch_combine_fwd(int dtype, int D, const Params& a, hipStream_t st) {
  DISPATCH_DTYPE_D(dtype, D, return combine_fwd_t<ElemT, kD>(a, st));
  return hipErrorInvalidValue;
}

hipError_t launch_combine_gg_row(int dtype, int D, const Params& a, bool gdo, hipStream_t st) {
  DISPATCH_DTYPE_D(dtype, D, return combine_gg_row_t<ElemT, kD>(a, gdo, st));
  return hipErrorInvalidValue;
}

}  // namespace ttt
