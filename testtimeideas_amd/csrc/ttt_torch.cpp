// ttt_torch.cpp — torch binding of the forward, backward and double backward
// of the C ABI (include/ttt_attn.h): ttt_attn_fwd, then ttt_attn_bwd and
// ttt_attn_gg, or, with a split of each kernel family's own (tiles per
// workgroup; 0 lets the library choose), ttt_attn_bwd_dq + ttt_attn_bwd_dkdv
// and ttt_attn_gg_row + ttt_attn_gg_col.
//
// The ctypes binding (testtimeideas_amd/_lib.py) spends tens of microseconds
// of Python per call building views, problems and outputs; the autograd path
// of one grad-grad step makes three such calls.  This module does the same
// work in C++: it takes tensors with the head dim already padded (by the
// Python layer), copies any whose strides the C ABI does not take (ready),
// allocates outputs, statistics and the workspace with torch's caching
// allocator on the tensors' device, and calls the C entry points on torch's
// current HIP stream.  A nonzero status raises
// RuntimeError with the library's message.  No kernel runs here and nothing
// falls back: the C ABI is the only compute path.
#include <torch/extension.h>
#include <c10/hip/HIPStream.h>

#include <algorithm>
#include <string>
#include <cstring>
#include <vector>

#include "../../include/ttt_attn.h"

namespace {

int32_t dtype_code(const at::Tensor& t) {
  switch (t.scalar_type()) {
    case at::kHalf: return TTT_F16;
    case at::kBFloat16: return TTT_BF16;
    case at::kFloat: return TTT_F32;
    default: TORCH_CHECK(false, "unsupported dtype ", t.scalar_type(), "; expected float16, bfloat16 or float32");
  }
  return -1;
}

ttt_view view_of(const at::Tensor& t) {
  ttt_view v;
  v.data = t.data_ptr();
  v.stride_b = t.stride(0);
  v.stride_h = t.stride(1);
  v.stride_t = t.stride(2);
  return v;
}

// `t` itself when the C ABI takes it as it is (unit last stride, a positive
// T stride, 16-byte aligned base and B/H/T strides), else a contiguous copy
// (fresh strides, so a size-1 dimension's stride is positive too).
at::Tensor ready(const at::Tensor& t) {
  const int64_t eb = t.element_size();
  const bool ok = (t.stride(3) == 1 || t.size(3) <= 1) && t.stride(2) > 0 &&
                  reinterpret_cast<uintptr_t>(t.data_ptr()) % 16 == 0 && (t.stride(0) * eb) % 16 == 0 &&
                  (t.stride(1) * eb) % 16 == 0 && (t.stride(2) * eb) % 16 == 0;
  return ok ? t : at::empty(t.sizes(), t.options()).copy_(t);
}

c10::optional<at::Tensor> ready(const c10::optional<at::Tensor>& t) {
  if (!t || !t->defined()) return t;
  return ready(*t);
}

ttt_view none_view() {
  ttt_view v;
  v.data = nullptr;
  v.stride_b = v.stride_h = v.stride_t = 0;
  return v;
}

// The problem of [B,H,T,D] tensor x with the mask fields.
ttt_problem problem_of(const at::Tensor& x, bool causal, double scale, int64_t split_chunk, int64_t window,
                       int64_t window_kind, const c10::optional<at::Tensor>& bias, int64_t block_rows = 0) {
  ttt_problem pr;
  std::memset(&pr, 0, sizeof(pr));
  pr.dtype = dtype_code(x);
  pr.causal = causal ? 1 : 0;
  pr.batch = x.size(0);
  pr.heads = x.size(1);
  pr.seqlen = x.size(2);
  pr.head_dim = x.size(3);
  pr.scale = static_cast<float>(scale);
  pr.split_chunk = static_cast<int32_t>(split_chunk);
  pr.window = static_cast<int32_t>(window);
  pr.window_kind = static_cast<int32_t>(window_kind);
  pr.bias = (bias && bias->defined()) ? view_of(*bias) : none_view();
  pr.block_rows = static_cast<int32_t>(block_rows);
  return pr;
}

void check(int rc, const char* what) {
  TORCH_CHECK(rc == 0, what, " failed (status ", rc, "): ", ttt_last_error());
}

at::Tensor stats_of(const at::Tensor& x) {
  return at::empty({x.size(0), x.size(1), x.size(2)}, x.options().dtype(at::kFloat));
}

// [B,H,T,T] P with rows padded to 8 elements (the kernels read rows in runs of 8).
at::Tensor alloc_p(const at::Tensor& x) {
  const int64_t t = x.size(2), tp = (t + 7) / 8 * 8;
  at::Tensor buf = at::empty({x.size(0), x.size(1), t, tp}, x.options());
  return tp == t ? buf : buf.narrow(3, 0, t);
}

int64_t workspace_size(const ttt_problem& pr, int32_t entry, bool gdo) {
  const int64_t n = ttt_attn_workspace_size(&pr, entry, gdo ? 1 : 0);
  TORCH_CHECK(n >= 0, "ttt_attn_workspace_size failed: ", ttt_last_error());
  return n;
}

at::Tensor workspace(const ttt_problem& pr, int32_t entry, bool gdo, const at::Tensor& like, int64_t* bytes) {
  const int64_t n = workspace_size(pr, entry, gdo);
  *bytes = n;
  return n > 0 ? at::empty({n}, like.options().dtype(at::kByte)) : at::Tensor();
}

// One workspace for two launches in stream order (the second starts after
// the first, its combine included, has finished with it).
at::Tensor workspace2(const ttt_problem& pr0, int32_t e0, const ttt_problem& pr1, int32_t e1, bool gdo,
                      const at::Tensor& like, int64_t* bytes) {
  const int64_t n = std::max(workspace_size(pr0, e0, gdo), workspace_size(pr1, e1, gdo));
  *bytes = n;
  return n > 0 ? at::empty({n}, like.options().dtype(at::kByte)) : at::Tensor();
}

void* ptr_or_null(const at::Tensor& t) { return t.defined() ? t.data_ptr() : nullptr; }

void* stream_of(const at::Tensor& x) {
  return static_cast<void*>(c10::hip::getCurrentHIPStream(x.device().index()).stream());
}

// Forward: (O, LSE, P or None).  Replaces TritonAttentionFn.forward's launches.
std::vector<at::Tensor> fwd(const at::Tensor& q_, const at::Tensor& k_, const at::Tensor& v_, bool causal,
                            double scale, bool want_p, int64_t split_chunk, int64_t window, int64_t window_kind,
                            const c10::optional<at::Tensor>& bias, int64_t block_rows) {
  const at::Tensor q = ready(q_), k = ready(k_), v = ready(v_);
  const ttt_problem pr = problem_of(q, causal, scale, split_chunk, window, window_kind, bias, block_rows);
  at::Tensor o = at::empty(q.sizes(), q.options());
  at::Tensor lse = stats_of(q);
  at::Tensor p = want_p ? alloc_p(q) : at::Tensor();
  int64_t wsb = 0;
  at::Tensor ws = workspace(pr, want_p ? TTT_ENTRY_FWD_P : TTT_ENTRY_FWD, false, q, &wsb);
  const ttt_view vq = view_of(q), vk = view_of(k), vv = view_of(v), vo = view_of(o);
  const ttt_view vp = want_p ? view_of(p) : none_view();
  check(ttt_attn_fwd(&pr, &vq, &vk, &vv, &vo, lse.data_ptr<float>(), want_p ? &vp : nullptr, ptr_or_null(ws), wsb,
                     stream_of(q)),
        "ttt_attn_fwd");
  return {o, lse, p};
}

// First backward: (dQ, dK, dV, D).  split_dq, split_dkdv: each family's split.
std::vector<at::Tensor> bwd(const at::Tensor& q_, const at::Tensor& k_, const at::Tensor& v_, const at::Tensor& o_,
                            const at::Tensor& dout_, const at::Tensor& lse, const c10::optional<at::Tensor>& p,
                            bool causal, double scale, int64_t split_dq, int64_t split_dkdv, int64_t window,
                            int64_t window_kind, const c10::optional<at::Tensor>& bias) {
  const at::Tensor q = ready(q_), k = ready(k_), v = ready(v_), o = ready(o_), dout = ready(dout_);
  const ttt_problem pq = problem_of(q, causal, scale, split_dq, window, window_kind, bias);
  const ttt_problem pk = problem_of(q, causal, scale, split_dkdv, window, window_kind, bias);
  at::Tensor dq = at::empty(q.sizes(), q.options());
  at::Tensor dk = at::empty(k.sizes(), k.options());
  at::Tensor dv = at::empty(v.sizes(), v.options());
  at::Tensor rowsum = stats_of(q);
  int64_t wsb = 0;
  at::Tensor ws = workspace2(pq, TTT_ENTRY_BWD_DQ, pk, TTT_ENTRY_BWD_DKDV, false, q, &wsb);
  const bool lp = p && p->defined();
  const ttt_view vq = view_of(q), vk = view_of(k), vv = view_of(v), vo = view_of(o), vdo = view_of(dout);
  const ttt_view vp = lp ? view_of(*p) : none_view();
  const ttt_view vdq = view_of(dq), vdk = view_of(dk), vdv = view_of(dv);
  void* st = stream_of(q);
  float* rs = rowsum.data_ptr<float>();
  check(ttt_attn_bwd_dq(&pq, &vq, &vk, &vv, &vo, &vdo, lse.data_ptr<float>(), lp ? &vp : nullptr, nullptr, rs, &vdq,
                        ptr_or_null(ws), wsb, st),
        "ttt_attn_bwd_dq");
  check(ttt_attn_bwd_dkdv(&pk, &vq, &vk, &vv, &vdo, lse.data_ptr<float>(), lp ? &vp : nullptr, rs, &vdk, &vdv,
                          ptr_or_null(ws), wsb, st),
        "ttt_attn_bwd_dkdv");
  return {dq, dk, dv, rowsum};
}

// The same through ttt_attn_bwd when both families take the library's split:
// the dK/dV launch then also finishes dQ's split blocks.
std::vector<at::Tensor> bwd_fused(const at::Tensor& q_, const at::Tensor& k_, const at::Tensor& v_,
                                  const at::Tensor& o_, const at::Tensor& dout_, const at::Tensor& lse,
                                  const c10::optional<at::Tensor>& p, bool causal, double scale, int64_t window,
                                  int64_t window_kind, const c10::optional<at::Tensor>& bias) {
  const at::Tensor q = ready(q_), k = ready(k_), v = ready(v_), o = ready(o_), dout = ready(dout_);
  const ttt_problem pr = problem_of(q, causal, scale, 0, window, window_kind, bias);
  at::Tensor dq = at::empty(q.sizes(), q.options());
  at::Tensor dk = at::empty(k.sizes(), k.options());
  at::Tensor dv = at::empty(v.sizes(), v.options());
  at::Tensor rowsum = stats_of(q);
  int64_t wsb = 0;
  at::Tensor ws = workspace(pr, TTT_ENTRY_BWD, false, q, &wsb);
  const bool lp = p && p->defined();
  const ttt_view vq = view_of(q), vk = view_of(k), vv = view_of(v), vo = view_of(o), vdo = view_of(dout);
  const ttt_view vp = lp ? view_of(*p) : none_view();
  const ttt_view vdq = view_of(dq), vdk = view_of(dk), vdv = view_of(dv);
  check(ttt_attn_bwd(&pr, &vq, &vk, &vv, &vo, &vdo, lse.data_ptr<float>(), lp ? &vp : nullptr,
                     rowsum.data_ptr<float>(), &vdq, &vdk, &vdv, ptr_or_null(ws), wsb, stream_of(q)),
        "ttt_attn_bwd");
  return {dq, dk, dv, rowsum};
}

// Double backward: (GQ, GK, GV, GdO or None).  dq: the first backward's dQ,
// or None (ttt_attn_gg_row).
std::vector<at::Tensor> gg(const at::Tensor& q_, const at::Tensor& k_, const at::Tensor& v_, const at::Tensor& dout_,
                           const at::Tensor& lse, const c10::optional<at::Tensor>& p, const at::Tensor& rowsum,
                           const c10::optional<at::Tensor>& dq_, const at::Tensor& gq_, const at::Tensor& gk_,
                           const at::Tensor& gv_, bool causal, double scale, bool want_gdo, int64_t split_row,
                           int64_t split_col, int64_t window, int64_t window_kind,
                           const c10::optional<at::Tensor>& bias) {
  const at::Tensor q = ready(q_), k = ready(k_), v = ready(v_), dout = ready(dout_);
  const at::Tensor gq = ready(gq_), gk = ready(gk_), gv = ready(gv_);
  const c10::optional<at::Tensor> dq = ready(dq_);
  const ttt_problem pr = problem_of(q, causal, scale, split_row, window, window_kind, bias);
  const ttt_problem pc = problem_of(q, causal, scale, split_col, window, window_kind, bias);
  at::Tensor gq_out = at::empty(q.sizes(), q.options());
  at::Tensor gk_out = at::empty(k.sizes(), k.options());
  at::Tensor gv_out = at::empty(v.sizes(), v.options());
  at::Tensor gdo = want_gdo ? at::empty(dout.sizes(), dout.options()) : at::Tensor();
  at::Tensor e = stats_of(q), f = stats_of(q);
  int64_t wsb = 0;
  at::Tensor ws = workspace2(pr, TTT_ENTRY_GG_ROW, pc, TTT_ENTRY_GG_COL, want_gdo, q, &wsb);
  const bool lp = p && p->defined();
  const ttt_view vq = view_of(q), vk = view_of(k), vv = view_of(v), vdo = view_of(dout);
  const ttt_view vp = lp ? view_of(*p) : none_view();
  const ttt_view vgq = view_of(gq), vgk = view_of(gk), vgv = view_of(gv);
  const ttt_view ogq = view_of(gq_out), ogk = view_of(gk_out), ogv = view_of(gv_out);
  const ttt_view ogdo = want_gdo ? view_of(gdo) : none_view();
  const bool ldq = dq && dq->defined();
  const ttt_view vdq = ldq ? view_of(*dq) : none_view();
  void* st = stream_of(q);
  const float* rs = rowsum.data_ptr<float>();
  check(ttt_attn_gg_row(&pr, &vq, &vk, &vv, &vdo, lse.data_ptr<float>(), lp ? &vp : nullptr, rs,
                        ldq ? &vdq : nullptr, &vgq, &vgk, &vgv, &ogq, want_gdo ? &ogdo : nullptr,
                        e.data_ptr<float>(), f.data_ptr<float>(), ptr_or_null(ws), wsb, st),
        "ttt_attn_gg_row");
  check(ttt_attn_gg_col(&pc, &vq, &vk, &vv, &vdo, lse.data_ptr<float>(), lp ? &vp : nullptr, rs,
                        e.data_ptr<float>(), f.data_ptr<float>(), &vgq, &vgk, &vgv, &ogk, &ogv, ptr_or_null(ws), wsb,
                        st),
        "ttt_attn_gg_col");
  return {gq_out, gk_out, gv_out, gdo};
}

// The same through ttt_attn_gg when both passes take the library's split:
// the column launch then also finishes the row pass's split blocks.
std::vector<at::Tensor> gg_fused(const at::Tensor& q_, const at::Tensor& k_, const at::Tensor& v_,
                                 const at::Tensor& dout_, const at::Tensor& lse, const c10::optional<at::Tensor>& p,
                                 const at::Tensor& rowsum, const c10::optional<at::Tensor>& dq_,
                                 const at::Tensor& gq_, const at::Tensor& gk_, const at::Tensor& gv_, bool causal,
                                 double scale, bool want_gdo, int64_t window, int64_t window_kind,
                                 const c10::optional<at::Tensor>& bias) {
  const at::Tensor q = ready(q_), k = ready(k_), v = ready(v_), dout = ready(dout_);
  const at::Tensor gq = ready(gq_), gk = ready(gk_), gv = ready(gv_);
  const c10::optional<at::Tensor> dq = ready(dq_);
  const ttt_problem pr = problem_of(q, causal, scale, 0, window, window_kind, bias);
  at::Tensor gq_out = at::empty(q.sizes(), q.options());
  at::Tensor gk_out = at::empty(k.sizes(), k.options());
  at::Tensor gv_out = at::empty(v.sizes(), v.options());
  at::Tensor gdo = want_gdo ? at::empty(dout.sizes(), dout.options()) : at::Tensor();
  at::Tensor e = stats_of(q), f = stats_of(q);
  int64_t wsb = 0;
  at::Tensor ws = workspace(pr, TTT_ENTRY_GG, want_gdo, q, &wsb);
  const bool lp = p && p->defined();
  const ttt_view vq = view_of(q), vk = view_of(k), vv = view_of(v), vdo = view_of(dout);
  const ttt_view vp = lp ? view_of(*p) : none_view();
  const ttt_view vgq = view_of(gq), vgk = view_of(gk), vgv = view_of(gv);
  const ttt_view ogq = view_of(gq_out), ogk = view_of(gk_out), ogv = view_of(gv_out);
  const ttt_view ogdo = want_gdo ? view_of(gdo) : none_view();
  const bool ldq = dq && dq->defined();
  const ttt_view vdq = ldq ? view_of(*dq) : none_view();
  check(ttt_attn_gg(&pr, &vq, &vk, &vv, &vdo, lse.data_ptr<float>(), lp ? &vp : nullptr, rowsum.data_ptr<float>(),
                    ldq ? &vdq : nullptr, &vgq, &vgk, &vgv, &ogq, &ogk, &ogv, want_gdo ? &ogdo : nullptr,
                    e.data_ptr<float>(), f.data_ptr<float>(), ptr_or_null(ws), wsb, stream_of(q)),
        "ttt_attn_gg");
  return {gq_out, gk_out, gv_out, gdo};
}

}  // namespace

PYBIND11_MODULE(TORCH_EXTENSION_NAME, m) {
  m.doc() = "torch binding of the forward, backward and double backward of libttt_attn.so";
  m.def("fwd", &fwd, "forward: (O, LSE, P or None)");
  m.def("bwd", &bwd, "first backward: (dQ, dK, dV, D)");
  m.def("bwd_fused", &bwd_fused, "first backward in one entry call: (dQ, dK, dV, D)");
  m.def("gg", &gg, "double backward: (GQ, GK, GV, GdO or None)");
  m.def("gg_fused", &gg_fused, "double backward in one entry call: (GQ, GK, GV, GdO or None)");
}
