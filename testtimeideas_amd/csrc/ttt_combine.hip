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
  if (nch <= kBatch) {
    // One round of loads: every chunk's (m, l, acc), then the same max and
    // the same in-order sum as the two-round form below.
    float mk[kBatch], lk[kBatch];
    f32x4 xk[kBatch];
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      const int64_t k = p0 + min(u, nch - 1);
      mk[u] = a.ws_sc[k * 2 * kBlk + r];
      lk[u] = a.ws_sc[k * 2 * kBlk + kBlk + r];
      xk[u] = *reinterpret_cast<const f32x4*>(a.ws_acc + k * kBlk * D + part_off<D>(r, cs.d0));
    }
#pragma unroll
    for (int u = 0; u < kBatch; ++u) mm = fmaxf(mm, mk[u]);
    float ll = 0.f;
    f32x4 v = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int u = 0; u < kBatch; ++u)
      if (u < nch) {
        const float wk = fast_exp2(mk[u] - mm);
        ll += lk[u] * wk;
        v += wk * xk[u];
      }
    store_slot<T>(a.o, b, h, row, cs.d0, v * (1.f / ll));
    if (cs.d0 == 0) a.lse[(int64_t)bh * T_ + row] = (mm + __log2f(ll)) * kLn2;
    return;
  }
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
      xk[u] = *reinterpret_cast<const f32x4*>(a.ws_acc + k * kBlk * D + part_off<D>(r, cs.d0));
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
// Grad-grad row pass: E, F, GQ (and GdO) of the split blocks.
template <typename T, int D, bool GDO>
__global__ __launch_bounds__(kThreads) void k_combine_gg_row(Params a) {
  combine_gg_row_block<T, D, GDO>(a, blockIdx.x, blockIdx.y, true);
}

// E and F alone (one thread per row), for the fused double backward, whose
// column launch sums GQ (and GdO) in workgroups appended to its grid.  The
// same sums in the same order as combine_gg_row_block, so bitwise the same.
__global__ __launch_bounds__(kThreads) void k_combine_gg_ef(Params a) {
  const int T_ = a.T;
  const int nblk = (T_ + kBlk - 1) / kBlk;
  const int row = blockIdx.x * kThreads + threadIdx.x;
  const int bh = blockIdx.y;
  if (row >= T_) return;
  const int blk = row / kBlk, r = row % kBlk;
  const int nch = block_nch(a, blk, nblk, false);
  if (nch <= 1) return;
  float sc[3];
  sum_scalars<3>(sc, a.ws_sc, part_index(a, bh, nblk, blk, 0), nch, r);
  const float ev = sc[0], xv = sc[1], dv = sc[2];
  a.e[(int64_t)bh * T_ + row] = ev;
  // the dQ form: dv = X summed in fp32, F = dv - E D
  a.f[(int64_t)bh * T_ + row] = a.dq.p ? dv - ev * a.rowsum_in[(int64_t)bh * T_ + row] : xv - ev * dv;
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

hipError_t launch_combine_gg_ef(const Params& a, hipStream_t st) {
  dim3 grid((a.T + kThreads - 1) / kThreads, a.B * a.H);
  hipLaunchKernelGGL(k_combine_gg_ef, grid, dim3(kThreads), 0, st, a);
  return hipGetLastError();
}

hipError_t launch_combine_gg_row(int dtype, int D, const Params& a, bool gdo, hipStream_t st) {
  DISPATCH_DTYPE_D(dtype, D, return combine_gg_row_t<ElemT, kD>(a, gdo, st));
  return hipErrorInvalidValue;
}

}  // namespace ttt
