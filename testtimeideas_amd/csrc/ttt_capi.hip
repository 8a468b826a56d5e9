// ttt_capi.hip — the extern "C" entry points declared in include/ttt_attn.h.
// Validates every argument on the host before anything is enqueued (shapes,
// null pointers, 16-byte alignment of bases and row strides, grid limits),
// packs the kernel argument block and calls the per-family launchers.
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <cstring>

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
  return TTT_OK;
}

ttt::Params base_params(const ttt_problem* pr) {
  ttt::Params a;
  std::memset(&a, 0, sizeof(a));
  a.B = (int)pr->batch;
  a.H = (int)pr->heads;
  a.T = (int)pr->seqlen;
  a.causal = pr->causal;
  a.scale = pr->scale;
  a.scale_log2 = pr->scale * ttt::kLog2e;
  return a;
}

bool has_p(const ttt_view* p) { return p && p->data; }

int launched(hipError_t e, const char* what) {
  if (e != hipSuccess) return fail(TTT_ERR_LAUNCH, "%s: launch failed: %s", what, hipGetErrorString(e));
  return TTT_OK;
}

#define TRY(x)                   \
  do {                           \
    const int rc_ = (x);         \
    if (rc_ != TTT_OK) return rc_; \
  } while (0)

}  // namespace

extern "C" {

int ttt_version(void) { return 100; }

const char* ttt_last_error(void) { return g_err; }

int ttt_attn_fwd(const ttt_problem* pr, const ttt_view* q, const ttt_view* k, const ttt_view* v,
                 const ttt_view* o, float* lse, const ttt_view* p, void* stream) {
  TRY(check_problem(pr));
  ttt::Params a = base_params(pr);
  TRY(take_view(pr, q, "q", &a.q));
  TRY(take_view(pr, k, "k", &a.k));
  TRY(take_view(pr, v, "v", &a.v));
  TRY(take_view(pr, o, "o", &a.o));
  if (!lse) return fail(TTT_ERR_INVALID_ARGUMENT, "lse: null pointer");
  a.lse = lse;
  const bool wp = has_p(p);
  if (wp) TRY(take_view(pr, p, "p", &a.p));
  return launched(ttt::launch_fwd(pr->dtype, (int)pr->head_dim, a, wp, (hipStream_t)stream), "ttt_attn_fwd");
}

int ttt_attn_bwd_dq(const ttt_problem* pr, const ttt_view* q, const ttt_view* k, const ttt_view* v,
                    const ttt_view* o, const ttt_view* dout, const float* lse, const ttt_view* p,
                    const float* rowsum_in, float* rowsum_out, const ttt_view* dq, void* stream) {
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
  a.lse = const_cast<float*>(lse);
  a.rowsum_in = rowsum_in;
  a.rowsum_out = rowsum_out;
  if (!rowsum_in) TRY(take_view(pr, o, "o (needed to form D without rowsum_in)", &a.o));
  return launched(ttt::launch_bwd_dq(pr->dtype, (int)pr->head_dim, a, lp, (hipStream_t)stream),
                  "ttt_attn_bwd_dq");
}

int ttt_attn_bwd_dkdv(const ttt_problem* pr, const ttt_view* q, const ttt_view* k, const ttt_view* v,
                      const ttt_view* dout, const float* lse, const ttt_view* p, const float* rowsum,
                      const ttt_view* dk, const ttt_view* dv, void* stream) {
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
  a.lse = const_cast<float*>(lse);
  a.rowsum_in = rowsum;
  return launched(ttt::launch_bwd_dkdv(pr->dtype, (int)pr->head_dim, a, lp, dv_only, (hipStream_t)stream),
                  "ttt_attn_bwd_dkdv");
}

int ttt_attn_bwd(const ttt_problem* pr, const ttt_view* q, const ttt_view* k, const ttt_view* v,
                 const ttt_view* o, const ttt_view* dout, const float* lse, const ttt_view* p,
                 float* rowsum_out, const ttt_view* dq, const ttt_view* dk, const ttt_view* dv,
                 void* stream) {
  if (!rowsum_out) return fail(TTT_ERR_INVALID_ARGUMENT, "rowsum_out: null pointer");
  if (!dk || !dk->data) return fail(TTT_ERR_INVALID_ARGUMENT, "dk: null pointer");
  TRY(ttt_attn_bwd_dq(pr, q, k, v, o, dout, lse, p, nullptr, rowsum_out, dq, stream));
  return ttt_attn_bwd_dkdv(pr, q, k, v, dout, lse, p, rowsum_out, dk, dv, stream);
}

int ttt_attn_bwd_rowsum(const ttt_problem* pr, const ttt_view* p, const ttt_view* dout, const ttt_view* v,
                        float* rowsum, void* stream) {
  TRY(check_problem(pr));
  ttt::Params a = base_params(pr);
  TRY(take_view(pr, p, "p", &a.p));
  TRY(take_view(pr, dout, "dout", &a.dout));
  TRY(take_view(pr, v, "v", &a.v));
  if (!rowsum) return fail(TTT_ERR_INVALID_ARGUMENT, "rowsum: null pointer");
  a.rowsum_out = rowsum;
  return launched(ttt::launch_bwd_rowsum(pr->dtype, (int)pr->head_dim, a, (hipStream_t)stream),
                  "ttt_attn_bwd_rowsum");
}

int ttt_attn_gg_row(const ttt_problem* pr, const ttt_view* q, const ttt_view* k, const ttt_view* v,
                    const ttt_view* dout, const float* lse, const ttt_view* p, const float* rowsum,
                    const ttt_view* gq, const ttt_view* gk, const ttt_view* gv, const ttt_view* gq_out,
                    const ttt_view* gdout, float* e_out, float* f_out, void* stream) {
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
  if (!rowsum || !e_out || !f_out) return fail(TTT_ERR_INVALID_ARGUMENT, "rowsum/e_out/f_out: null pointer");
  a.lse = const_cast<float*>(lse);
  a.rowsum_in = rowsum;
  a.e = e_out;
  a.f = f_out;
  return launched(ttt::launch_gg_row(pr->dtype, (int)pr->head_dim, a, lp, gdo, (hipStream_t)stream),
                  "ttt_attn_gg_row");
}

int ttt_attn_gg_col(const ttt_problem* pr, const ttt_view* q, const ttt_view* k, const ttt_view* v,
                    const ttt_view* dout, const float* lse, const ttt_view* p, const float* rowsum,
                    const float* e_in, const float* f_in, const ttt_view* gq, const ttt_view* gk,
                    const ttt_view* gv, const ttt_view* gk_out, const ttt_view* gv_out, void* stream) {
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
  a.lse = const_cast<float*>(lse);
  a.rowsum_in = rowsum;
  a.e = const_cast<float*>(e_in);
  a.f = const_cast<float*>(f_in);
  return launched(ttt::launch_gg_col(pr->dtype, (int)pr->head_dim, a, lp, (hipStream_t)stream),
                  "ttt_attn_gg_col");
}

int ttt_attn_gg(const ttt_problem* pr, const ttt_view* q, const ttt_view* k, const ttt_view* v,
                const ttt_view* dout, const float* lse, const ttt_view* p, const float* rowsum,
                const ttt_view* gq, const ttt_view* gk, const ttt_view* gv, const ttt_view* gq_out,
                const ttt_view* gk_out, const ttt_view* gv_out, const ttt_view* gdout, float* e_buf,
                float* f_buf, void* stream) {
  TRY(ttt_attn_gg_row(pr, q, k, v, dout, lse, p, rowsum, gq, gk, gv, gq_out, gdout, e_buf, f_buf, stream));
  return ttt_attn_gg_col(pr, q, k, v, dout, lse, p, rowsum, e_buf, f_buf, gq, gk, gv, gk_out, gv_out, stream);
}

}  // extern "C"
