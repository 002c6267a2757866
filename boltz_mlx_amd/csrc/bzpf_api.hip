// C-ABI entry points (declared in include/bzpf.h): argument validation, dispatch to the launchers, error capture.
#include <cstdarg>
#include <cstdio>

#include "bzpf.h"
#include "bzpf_kernels.h"
#include "bzpf_layout.h"

namespace {

thread_local char g_err[512] = "";

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

int done(hipError_t e, const char* what) {
  if (e == hipSuccess) {
    g_err[0] = 0;
    return BZPF_OK;
  }
  return fail(BZPF_ELAUNCH, "%s: %s", what, hipGetErrorString(e));
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
bool dt_ok(int dt) { return dt == BZPF_F32 || dt == BZPF_F16; }
hipStream_t S(void* s) { return static_cast<hipStream_t>(s); }

}  // namespace

#define REQUIRE(cond, ...) \
  do {                     \
    if (!(cond)) return fail(BZPF_EINVAL, __VA_ARGS__); \
  } while (0)
#define REQUIRE_PTR(p) REQUIRE((p) != nullptr && aligned16(p), "%s: %s must be a non-null 16-byte aligned pointer", __func__, #p)

extern "C" {

const char* bzpf_version(void) { return "bzpf 0.1.0 (gfx950)"; }

const char* bzpf_last_error(void) { return g_err; }

int64_t bzpf_row_pitch(int64_t N) { return bzpf::row_pitch(N); }

int bzpf_layernorm(const void* x, int x_dt, const float* w, const float* b, float eps, void* y, int y_dt,
                   int64_t rows, int D, void* stream) {
  REQUIRE_PTR(x);
  REQUIRE_PTR(y);
  REQUIRE(dt_ok(x_dt) && dt_ok(y_dt), "bzpf_layernorm: bad dtype %d/%d", x_dt, y_dt);
  REQUIRE(D % 64 == 0 && D >= 64 && D <= 1024 && (D / 64 <= 6 || D / 64 == 8 || D / 64 == 12 || D / 64 == 16),
          "bzpf_layernorm: unsupported D=%d", D);
  REQUIRE(rows >= 0, "bzpf_layernorm: rows < 0");
  if (rows == 0) return BZPF_OK;
  return done(bzpf::launch_layernorm(x, x_dt, w, b, eps, y, y_dt, rows, D, S(stream)), "bzpf_layernorm");
}

int bzpf_count_nonfinite(const void* x, int dt, int64_t n, int* count, void* stream) {
  REQUIRE(count != nullptr, "bzpf_count_nonfinite: count is NULL");
  REQUIRE(dt_ok(dt), "bzpf_count_nonfinite: bad dtype %d", dt);
  REQUIRE(n >= 0, "bzpf_count_nonfinite: n < 0");
  if (n == 0) return BZPF_OK;
  REQUIRE_PTR(x);
  return done(bzpf::launch_count_nonfinite(x, dt, n, count, S(stream)), "bzpf_count_nonfinite");
}

int bzpf_add_ln(float* z, const void* y, int y_dt, float y_scale, int trans_y, const float* w, const float* b,
                float eps, void* ln, int ln_dt, int trans_out, int64_t N, int D, void* stream) {
  REQUIRE_PTR(z);
  REQUIRE_PTR(y);
  REQUIRE(ln == nullptr || aligned16(ln), "bzpf_add_ln: ln misaligned");
  REQUIRE(dt_ok(y_dt) && dt_ok(ln_dt), "bzpf_add_ln: bad dtype");
  REQUIRE(D % 64 == 0 && D >= 64 && D <= 384 && D != 320, "bzpf_add_ln: unsupported D=%d", D);
  REQUIRE(N >= 0, "bzpf_add_ln: N < 0");
  if (N == 0) return BZPF_OK;
  return done(bzpf::launch_add_ln(z, y, y_dt, y_scale, trans_y, w, b, eps, ln, ln_dt, trans_out, N, D, S(stream)),
              "bzpf_add_ln");
}

int bzpf_trimul_proj(const void* xn, const void* w_pg, const float* pair_mask, float scale, int incoming, void* ab,
                     int dt, int64_t N, int64_t ld, int D, void* stream) {
  REQUIRE_PTR(xn);
  REQUIRE_PTR(w_pg);
  REQUIRE_PTR(ab);
  REQUIRE(pair_mask != nullptr, "bzpf_trimul_proj: pair_mask is NULL");
  REQUIRE(dt_ok(dt), "bzpf_trimul_proj: bad dtype %d", dt);
  REQUIRE(D == 128, "bzpf_trimul_proj: D must be 128 (got %d)", D);
  REQUIRE(N >= 1 && ld == bzpf_row_pitch(N), "bzpf_trimul_proj: N=%lld ld=%lld (ld must be bzpf_row_pitch(N))",
          (long long)N, (long long)ld);
  return done(bzpf::launch_trimul_proj(xn, w_pg, pair_mask, scale, incoming, ab, dt, N, ld, S(stream)),
              "bzpf_trimul_proj");
}

int bzpf_trimul_contract(const void* ab, void* o, int dt, int64_t N, int64_t ld, int D, int64_t k_len,
                         void* stream) {
  REQUIRE_PTR(ab);
  REQUIRE_PTR(o);
  REQUIRE(dt_ok(dt), "bzpf_trimul_contract: bad dtype %d", dt);
  REQUIRE(D >= 1 && D <= 65535, "bzpf_trimul_contract: bad D=%d", D);
  REQUIRE(N >= 1 && ld == bzpf_row_pitch(N), "bzpf_trimul_contract: N=%lld ld=%lld", (long long)N, (long long)ld);
  return done(bzpf::launch_trimul_contract(ab, o, dt, N, ld, k_len, D, S(stream)), "bzpf_trimul_contract");
}

int bzpf_trimul_tail(const void* o, const float* norm_out_w, const float* norm_out_b, float eps_out,
                     const void* w_po, const void* xn, const void* w_go, float* z, int accumulate,
                     const float* next_w, const float* next_b, float next_eps, void* xn_next, int dt, int64_t N,
                     int64_t ld, int D, void* stream) {
  REQUIRE_PTR(o);
  REQUIRE_PTR(w_po);
  REQUIRE_PTR(xn);
  REQUIRE_PTR(w_go);
  REQUIRE_PTR(z);
  REQUIRE(norm_out_w && norm_out_b, "bzpf_trimul_tail: norm_out weight/bias required");
  REQUIRE(next_w == nullptr || (next_b != nullptr && xn_next != nullptr),
          "bzpf_trimul_tail: next LN needs next_b and xn_next");
  REQUIRE(dt_ok(dt), "bzpf_trimul_tail: bad dtype %d", dt);
  REQUIRE(D == 128, "bzpf_trimul_tail: D must be 128 (got %d)", D);
  REQUIRE(N >= 1 && ld == bzpf_row_pitch(N), "bzpf_trimul_tail: N=%lld ld=%lld", (long long)N, (long long)ld);
  return done(bzpf::launch_trimul_tail(o, norm_out_w, norm_out_b, eps_out, w_po, xn, w_go, z, accumulate, next_w,
                                       next_b, next_eps, xn_next, dt, N, ld, S(stream)),
              "bzpf_trimul_tail");
}

int bzpf_triattn_proj(const void* xn, const void* w, int trans, float q_scale, float bias_scale, void* qkg, void* vt,
                      void* tri_bias, int dt, int64_t N, int64_t ldk, int D, int H, int C, void* stream) {
  REQUIRE_PTR(xn);
  REQUIRE_PTR(w);
  REQUIRE_PTR(qkg);
  REQUIRE(vt != nullptr && tri_bias != nullptr, "bzpf_triattn_proj: NULL pointer");
  REQUIRE(dt_ok(dt), "bzpf_triattn_proj: bad dtype %d", dt);
  REQUIRE(D == 128 && H >= 1 && H * C == 128 && (C == 16 || C == 32 || C == 64),
          "bzpf_triattn_proj: need D = H*C = 128, C in {16,32,64} (D=%d H=%d C=%d)", D, H, C);
  REQUIRE(N >= 1 && ldk == bzpf_row_pitch(N), "bzpf_triattn_proj: N=%lld ldk=%lld (ldk must be bzpf_row_pitch(N))",
          (long long)N, (long long)ldk);
  return done(bzpf::launch_triattn_proj(xn, w, trans, q_scale, bias_scale, qkg, vt, tri_bias, dt, N, ldk, H, C,
                                        S(stream)),
              "bzpf_triattn_proj");
}

int bzpf_triattn_core(const void* qkg, const void* vt, const void* tri_bias, const float* mask, int64_t mask_si,
                      int64_t mask_sk, float inf, void* out, int dt, int64_t N, int64_t ldk, int H, int C, int impl,
                      void* stream) {
  REQUIRE_PTR(qkg);
  REQUIRE_PTR(vt);
  REQUIRE_PTR(tri_bias);
  REQUIRE_PTR(out);
  REQUIRE(mask != nullptr, "bzpf_triattn_core: mask is NULL");
  REQUIRE(dt_ok(dt), "bzpf_triattn_core: bad dtype %d", dt);
  REQUIRE(H >= 1 && H <= 65535 && (C == 16 || C == 32 || C == 64), "bzpf_triattn_core: H=%d C=%d", H, C);
  REQUIRE(N >= 1 && N <= 65535 && ldk == bzpf_row_pitch(N), "bzpf_triattn_core: N=%lld ldk=%lld", (long long)N,
          (long long)ldk);
  REQUIRE(impl >= 0 && impl <= 2, "bzpf_triattn_core: impl must be 0 (auto), 1 (VALU) or 2 (MFMA)");
  REQUIRE(impl != 2 || (dt == BZPF_F16 && C == 32), "bzpf_triattn_core: the MFMA core needs fp16 and C = 32");
  return done(bzpf::launch_triattn_core(qkg, vt, tri_bias, mask, mask_si, mask_sk, inf, out, dt, N, ldk, H, C, impl,
                                        S(stream)),
              "bzpf_triattn_core");
}

int bzpf_linear_resid_ln(const void* x, const void* w, int trans, float* z, int accumulate, const float* next_w,
                         const float* next_b, float next_eps, void* xn_next, int dt, int64_t N, int D, void* stream) {
  REQUIRE_PTR(x);
  REQUIRE_PTR(w);
  REQUIRE_PTR(z);
  REQUIRE(next_w == nullptr || (next_b != nullptr && xn_next != nullptr),
          "bzpf_linear_resid_ln: next LN needs next_b and xn_next");
  REQUIRE(dt_ok(dt), "bzpf_linear_resid_ln: bad dtype %d", dt);
  REQUIRE(D == 128, "bzpf_linear_resid_ln: D must be 128 (got %d)", D);
  REQUIRE(N >= 1, "bzpf_linear_resid_ln: N < 1");
  return done(bzpf::launch_linear_resid_ln(x, w, trans, z, accumulate, next_w, next_b, next_eps, xn_next, dt, N,
                                           S(stream)),
              "bzpf_linear_resid_ln");
}

int bzpf_transition(const void* xn, const void* w12, const void* w3, float* z, int accumulate, const float* next_w,
                    const float* next_b, float next_eps, void* xn_next, int dt, int64_t rows, int D, int hidden,
                    void* stream) {
  REQUIRE_PTR(xn);
  REQUIRE_PTR(w12);
  REQUIRE_PTR(w3);
  REQUIRE_PTR(z);
  REQUIRE(next_w == nullptr || (next_b != nullptr && xn_next != nullptr),
          "bzpf_transition: next LN needs next_b and xn_next");
  REQUIRE(dt_ok(dt), "bzpf_transition: bad dtype %d", dt);
  REQUIRE(D == 128 && hidden >= 64 && hidden % 64 == 0, "bzpf_transition: need D=128, hidden %% 64 == 0 (D=%d H=%d)",
          D, hidden);
  REQUIRE(rows >= 0, "bzpf_transition: rows < 0");
  if (rows == 0) return BZPF_OK;
  return done(bzpf::launch_transition(xn, w12, w3, z, accumulate, next_w, next_b, next_eps, xn_next, dt, rows, hidden,
                                      S(stream)),
              "bzpf_transition");
}

int bzpf_transition_pb(const void* xn, const void* w12, const void* w3, float* z, int accumulate, const float* next_w,
                       const float* next_b, float next_eps, void* xn_next, const void* pb_w, const float* pb_lnw,
                       const float* pb_lnb, float pb_eps, void* pb_out, int pb_heads, int dt, int64_t rows, int D,
                       int hidden, void* stream) {
  REQUIRE_PTR(xn);
  REQUIRE_PTR(w12);
  REQUIRE_PTR(w3);
  REQUIRE_PTR(z);
  REQUIRE(pb_w != nullptr && pb_lnw != nullptr && pb_lnb != nullptr && pb_out != nullptr,
          "bzpf_transition_pb: NULL pair-bias pointer");
  REQUIRE(next_w == nullptr || (next_b != nullptr && xn_next != nullptr),
          "bzpf_transition_pb: next LN needs next_b and xn_next");
  REQUIRE(dt_ok(dt), "bzpf_transition_pb: bad dtype %d", dt);
  REQUIRE(D == 128 && hidden >= 64 && hidden % 64 == 0,
          "bzpf_transition_pb: need D=128, hidden %% 64 == 0 (D=%d H=%d)", D, hidden);
  REQUIRE(pb_heads >= 1 && pb_heads <= 16, "bzpf_transition_pb: 1 <= heads <= 16 (got %d)", pb_heads);
  REQUIRE(rows >= 0, "bzpf_transition_pb: rows < 0");
  if (rows == 0) return BZPF_OK;
  return done(bzpf::launch_transition_pb(xn, w12, w3, z, accumulate, next_w, next_b, next_eps, xn_next, pb_w, pb_lnw,
                                         pb_lnb, pb_eps, pb_out, pb_heads, dt, rows, hidden, S(stream)),
              "bzpf_transition_pb");
}

int bzpf_attn_out_transition(const void* o, const void* w_o, int trans, const float* ln_w, const float* ln_b,
                             float ln_eps, const void* w12, const void* w3, float* z, const float* next_w,
                             const float* next_b, float next_eps, void* xn_next, const void* pb_w,
                             const float* pb_lnw, const float* pb_lnb, float pb_eps, void* pb_out, int pb_heads, int dt,
                             int64_t N, int D, int hidden, void* stream) {
  REQUIRE_PTR(o);
  REQUIRE_PTR(w_o);
  REQUIRE(ln_w != nullptr && ln_b != nullptr, "bzpf_attn_out_transition: NULL LayerNorm pointer");
  REQUIRE_PTR(w12);
  REQUIRE_PTR(w3);
  REQUIRE_PTR(z);
  REQUIRE(next_w == nullptr || (next_b != nullptr && xn_next != nullptr),
          "bzpf_attn_out_transition: next LN needs next_b and xn_next");
  REQUIRE(pb_w == nullptr || (pb_lnw != nullptr && pb_lnb != nullptr && pb_out != nullptr),
          "bzpf_attn_out_transition: pair bias needs pb_lnw, pb_lnb and pb_out");
  REQUIRE(pb_w == nullptr || (pb_heads >= 1 && pb_heads <= 16), "bzpf_attn_out_transition: 1 <= heads <= 16 (got %d)",
          pb_heads);
  REQUIRE(dt == BZPF_F16, "bzpf_attn_out_transition: fp16 only (dt=%d)", dt);
  REQUIRE(D == 128 && hidden >= 64 && hidden % 64 == 0,
          "bzpf_attn_out_transition: need D=128, hidden %% 64 == 0 (D=%d H=%d)", D, hidden);
  REQUIRE(N >= 0 && N <= 46340, "bzpf_attn_out_transition: bad N=%lld", (long long)N);
  if (N == 0) return BZPF_OK;
  return done(bzpf::launch_attn_out_transition(o, w_o, trans, ln_w, ln_b, ln_eps, w12, w3, z, next_w, next_b, next_eps,
                                               xn_next, pb_w, pb_lnw, pb_lnb, pb_eps, pb_out, pb_heads, N, hidden,
                                               S(stream)),
              "bzpf_attn_out_transition");
}

int bzpf_linear(const void* x, const void* w, const float* bias, void* y, int dt, int y_dt, int64_t rows, int K,
                int M, int accumulate, void* stream) {
  REQUIRE_PTR(x);
  REQUIRE_PTR(w);
  REQUIRE(y != nullptr, "bzpf_linear: y is NULL");
  REQUIRE(dt_ok(dt) && dt_ok(y_dt), "bzpf_linear: bad dtype");
  REQUIRE(K >= 8 && K % 8 == 0 && M >= 1, "bzpf_linear: need K %% 8 == 0, M >= 1 (K=%d M=%d)", K, M);
  REQUIRE(!accumulate || y_dt == BZPF_F32, "bzpf_linear: accumulate needs an fp32 y");
  REQUIRE(rows >= 0, "bzpf_linear: rows < 0");
  if (rows == 0) return BZPF_OK;
  return done(bzpf::launch_linear(x, w, bias, y, dt, y_dt, rows, K, M, accumulate ? 1 : 0, S(stream)), "bzpf_linear");
}

int bzpf_linear_residual(const void* x, const void* w, const float* bias, const float* res, int64_t ld_res, float* y,
                         int dt, int64_t rows, int K, int M, void* stream) {
  REQUIRE_PTR(x);
  REQUIRE_PTR(w);
  REQUIRE(res != nullptr && y != nullptr, "bzpf_linear_residual: NULL pointer");
  REQUIRE(dt_ok(dt), "bzpf_linear_residual: bad dtype");
  REQUIRE(K >= 8 && K % 8 == 0 && M >= 1, "bzpf_linear_residual: need K %% 8 == 0, M >= 1 (K=%d M=%d)", K, M);
  REQUIRE(ld_res >= M && ld_res % 4 == 0 && reinterpret_cast<uintptr_t>(res) % 16 == 0,
          "bzpf_linear_residual: res must be 16-byte aligned with a pitch >= M, a multiple of 4 (ld_res=%lld)",
          (long long)ld_res);
  REQUIRE(rows >= 0, "bzpf_linear_residual: rows < 0");
  if (rows == 0) return BZPF_OK;
  if (bzpf::gemm_nt_ok(dt, x, w, bias, y, rows, K, M, res, ld_res))
    return done(bzpf::launch_gemm_nt(x, w, bias, y, dt, BZPF_F32, rows, K, M, 3, res, ld_res, rows, S(stream)),
                "bzpf_linear_residual");
  // other shapes: the residual copied into y, then the accumulating layer (the same sums)
  const hipError_t e = hipMemcpy2DAsync(y, (size_t)M * 4, res, (size_t)ld_res * 4, (size_t)M * 4, (size_t)rows,
                                        hipMemcpyDeviceToDevice, S(stream));
  if (e != hipSuccess) return done(e, "bzpf_linear_residual");
  return done(bzpf::launch_linear(x, w, bias, y, dt, BZPF_F32, rows, K, M, 1, S(stream)), "bzpf_linear_residual");
}

int bzpf_swiglu(const void* h, void* a, int dt, int64_t rows, int hidden, void* stream) {
  REQUIRE(h != nullptr && a != nullptr, "bzpf_swiglu: NULL pointer");
  REQUIRE(dt_ok(dt), "bzpf_swiglu: bad dtype");
  REQUIRE(rows >= 0 && hidden >= 1, "bzpf_swiglu: bad sizes");
  if (rows == 0) return BZPF_OK;
  return done(bzpf::launch_swiglu(h, a, dt, rows, hidden, S(stream)), "bzpf_swiglu");
}

int bzpf_linear_gated(const void* x, const void* w, const float* bias, const float* gate, int64_t ld_gate,
                      int64_t gate_rows, float* y, int dt, int64_t rows, int K, int M, void* stream) {
  REQUIRE_PTR(x);
  REQUIRE_PTR(w);
  REQUIRE(gate != nullptr && y != nullptr, "bzpf_linear_gated: NULL pointer");
  REQUIRE(dt_ok(dt), "bzpf_linear_gated: bad dtype");
  REQUIRE(K >= 8 && K % 8 == 0 && M >= 1, "bzpf_linear_gated: need K %% 8 == 0, M >= 1 (K=%d M=%d)", K, M);
  REQUIRE(rows >= 0 && gate_rows >= 1 && ld_gate >= M, "bzpf_linear_gated: bad sizes");
  if (rows == 0) return BZPF_OK;
  return done(bzpf::launch_linear_gated(x, w, bias, gate, ld_gate, gate_rows, y, dt, rows, K, M, S(stream)),
              "bzpf_linear_gated");
}

int bzpf_swiglu3(const void* h, void* a, int dt, int64_t rows, int hidden, void* stream) {
  REQUIRE(h != nullptr && a != nullptr, "bzpf_swiglu3: NULL pointer");
  REQUIRE(dt_ok(dt), "bzpf_swiglu3: bad dtype");
  REQUIRE(rows >= 0 && hidden >= 1, "bzpf_swiglu3: bad sizes");
  if (rows == 0) return BZPF_OK;
  return done(bzpf::launch_swiglu3(h, a, dt, rows, hidden, S(stream)), "bzpf_swiglu3");
}

int bzpf_adaln(const float* a, const float* scale, const float* shift, int64_t ld_cond, int64_t cond_rows, float eps,
               void* out, int out_dt, int64_t rows, int D, void* stream) {
  REQUIRE(a != nullptr && scale != nullptr && shift != nullptr && out != nullptr, "bzpf_adaln: NULL pointer");
  REQUIRE(dt_ok(out_dt), "bzpf_adaln: bad dtype");
  REQUIRE(D % 64 == 0 && D >= 64 && D <= 1024 && (D / 64 <= 4 || D / 64 == 6 || D / 64 == 8 || D / 64 == 12 ||
                                                  D / 64 == 16),
          "bzpf_adaln: unsupported D=%d", D);
  REQUIRE(rows >= 0 && cond_rows >= 1 && ld_cond >= D, "bzpf_adaln: bad sizes");
  if (rows == 0) return BZPF_OK;
  return done(bzpf::launch_adaln(a, scale, shift, ld_cond, cond_rows, eps, out, out_dt, rows, D, S(stream)),
              "bzpf_adaln");
}

int bzpf_seq_attention_batched(const void* q, const void* k, const void* v, const void* g, int64_t ld_in,
                               int64_t s_in, const void* bias, int64_t s_bias, int mult, const float* mask,
                               int64_t s_mask, float inf, void* out, int64_t ld_out, int64_t s_out, int dt, int bias_dt,
                               int n_samples, int64_t N, int H, int hd, void* stream) {
  REQUIRE(q && k && v && g && bias && mask && out, "bzpf_seq_attention: NULL pointer");
  REQUIRE(dt_ok(dt) && dt_ok(bias_dt), "bzpf_seq_attention: bad dtype");
  REQUIRE(hd == 16 || hd == 24 || hd == 32 || hd == 48 || hd == 64, "bzpf_seq_attention: hd=%d unsupported", hd);
  REQUIRE(H >= 1 && H <= 65535 && N >= 1 && ld_in >= (int64_t)H * hd && ld_out >= (int64_t)H * hd,
          "bzpf_seq_attention: bad sizes");
  REQUIRE(n_samples >= 1 && n_samples <= 65535 && mult >= 1 && s_in >= 0 && s_bias >= 0 && s_mask >= 0 && s_out >= 0,
          "bzpf_seq_attention: bad sample count or strides (S=%d mult=%d)", n_samples, mult);
  return done(bzpf::launch_seq_attention(q, k, v, g, ld_in, s_in, bias, s_bias, mult, mask, s_mask, inf, out, ld_out,
                                         s_out, dt, bias_dt, n_samples, N, H, hd, S(stream)),
              "bzpf_seq_attention");
}

int bzpf_seq_attention(const void* q, const void* k, const void* v, const void* g, int64_t ld_in, const void* bias,
                       const float* mask, float inf, void* out, int64_t ld_out, int dt, int bias_dt, int64_t N, int H,
                       int hd, void* stream) {
  return bzpf_seq_attention_batched(q, k, v, g, ld_in, 0, bias, 0, 1, mask, 0, inf, out, ld_out, 0, dt, bias_dt, 1, N,
                                    H, hd, stream);
}

int bzpf_linear_swiglu3(const void* x, const void* w, void* u, int64_t rows, int K, int H, void* stream) {
  REQUIRE(x && w && u, "bzpf_linear_swiglu3: NULL pointer");
  REQUIRE(aligned16(x) && aligned16(w) && reinterpret_cast<uintptr_t>(u) % 8 == 0,
          "bzpf_linear_swiglu3: x and w must be 16-byte aligned, u 8-byte aligned");
  REQUIRE(rows >= 1 && K >= 64 && K % 64 == 0 && K <= (1 << 22) && H >= 32 && H % 32 == 0,
          "bzpf_linear_swiglu3: need K %% 64 == 0, H %% 32 == 0 (rows=%lld K=%d H=%d)", (long long)rows, K, H);
  return done(bzpf::launch_gemm_swiglu_f16(x, w, u, rows, K, H, 3, S(stream)), "bzpf_linear_swiglu3");
}

int bzpf_linear_swiglu(const void* x, const void* w, void* u, int64_t rows, int K, int H, void* stream) {
  REQUIRE(x && w && u, "bzpf_linear_swiglu: NULL pointer");
  REQUIRE(aligned16(x) && aligned16(w) && reinterpret_cast<uintptr_t>(u) % 8 == 0,
          "bzpf_linear_swiglu: x and w must be 16-byte aligned, u 8-byte aligned");
  REQUIRE(rows >= 1 && K >= 64 && K % 64 == 0 && K <= (1 << 22) && H >= 32 && H % 32 == 0,
          "bzpf_linear_swiglu: need K %% 64 == 0, H %% 32 == 0 (rows=%lld K=%d H=%d)", (long long)rows, K, H);
  return done(bzpf::launch_gemm_swiglu_f16(x, w, u, rows, K, H, 2, S(stream)), "bzpf_linear_swiglu");
}

int bzpf_trimul_pack(const void* P, const float* mask, float scale, int incoming, void* ab, int dt, int64_t N,
                     int64_t ld, int D, void* stream) {
  REQUIRE(P && mask && ab, "bzpf_trimul_pack: NULL pointer");
  REQUIRE(dt_ok(dt), "bzpf_trimul_pack: bad dtype %d", dt);
  REQUIRE(N >= 1 && N <= 65535 && ld == bzpf_row_pitch(N), "bzpf_trimul_pack: N=%lld ld=%lld", (long long)N,
          (long long)ld);
  REQUIRE(D >= 1 && D <= 4096, "bzpf_trimul_pack: need 1 <= D <= 4096 (D=%d)", D);
  return done(bzpf::launch_trimul_pack(P, mask, scale, incoming, ab, dt, N, ld, D, S(stream)), "bzpf_trimul_pack");
}

int bzpf_channels_to_rows(const void* o, int o_dt, void* out, int out_dt, int64_t N, int64_t ld, int D,
                          void* stream) {
  REQUIRE(o && out, "bzpf_channels_to_rows: NULL pointer");
  REQUIRE(dt_ok(o_dt) && dt_ok(out_dt), "bzpf_channels_to_rows: bad dtype");
  REQUIRE(N >= 1 && N <= 65535 && ld == bzpf_row_pitch(N), "bzpf_channels_to_rows: N=%lld ld=%lld", (long long)N,
          (long long)ld);
  REQUIRE(D >= 1 && D <= 252, "bzpf_channels_to_rows: need 1 <= D <= 252 (D=%d)", D);
  return done(bzpf::launch_channels_to_rows(o, o_dt, out, out_dt, N, ld, D, S(stream)), "bzpf_channels_to_rows");
}

int bzpf_triattn_pack(const void* P, int trans, float q_scale, float bias_scale, void* qkg, void* vt, void* tri_bias,
                      int dt, int64_t N, int64_t ldk, int H, int C, void* stream) {
  REQUIRE(P && qkg && vt && tri_bias, "bzpf_triattn_pack: NULL pointer");
  REQUIRE(dt_ok(dt), "bzpf_triattn_pack: bad dtype %d", dt);
  REQUIRE(N >= 1 && N <= 65535 && ldk == bzpf_row_pitch(N), "bzpf_triattn_pack: N=%lld ldk=%lld", (long long)N,
          (long long)ldk);
  REQUIRE(H >= 1 && C >= 1 && H * C + H <= 252, "bzpf_triattn_pack: need H*C + H <= 252 (H=%d C=%d)", H, C);
  return done(bzpf::launch_triattn_pack(P, trans, q_scale, bias_scale, qkg, vt, tri_bias, dt, N, ldk, H, C,
                                        S(stream)),
              "bzpf_triattn_pack");
}

int bzpf_opm_split(const float* ab, int64_t ld_ab, const float* mask, void* planes, int n_seq, int N,
                   void* stream) {
  REQUIRE(ab && mask && planes, "bzpf_opm_split: NULL pointer");
  REQUIRE(reinterpret_cast<uintptr_t>(planes) % 16 == 0 && ld_ab >= 64,
          "bzpf_opm_split: planes must be 16-byte aligned and ab's row pitch >= 64 (ld_ab=%lld)", (long long)ld_ab);
  REQUIRE(n_seq >= 1 && n_seq <= 16 * 65535 && N >= 1 && (int64_t)N * 6144 <= INT32_MAX,
          "bzpf_opm_split: bad sizes (n_seq=%d N=%d)", n_seq, N);
  return done(bzpf::launch_opm_split(ab, ld_ab, mask, planes, n_seq, N, S(stream)), "bzpf_opm_split");
}

int bzpf_opm_ln_split(const float* m, const float* ln_w, const float* ln_b, float eps, const float* w_ab,
                      const float* mask, void* planes, int n_seq, int N, void* stream) {
  REQUIRE(m && ln_w && ln_b && w_ab && mask && planes, "bzpf_opm_ln_split: NULL pointer");
  REQUIRE(reinterpret_cast<uintptr_t>(m) % 16 == 0 && reinterpret_cast<uintptr_t>(w_ab) % 16 == 0 &&
              reinterpret_cast<uintptr_t>(ln_w) % 16 == 0 && reinterpret_cast<uintptr_t>(ln_b) % 16 == 0 &&
              reinterpret_cast<uintptr_t>(planes) % 16 == 0,
          "bzpf_opm_ln_split: m, w_ab, ln_w, ln_b and planes must be 16-byte aligned");
  REQUIRE(n_seq >= 1 && n_seq <= 16 * 65535 && N >= 1 && (int64_t)N * 6144 <= INT32_MAX,
          "bzpf_opm_ln_split: bad sizes (n_seq=%d N=%d)", n_seq, N);
  return done(bzpf::launch_opm_ln_split(m, ln_w, ln_b, eps, w_ab, mask, planes, n_seq, N, S(stream)),
              "bzpf_opm_ln_split");
}

int bzpf_opm_outer(const void* planes, const float* num, void* out, int out_dt, int n_seq, int N, int i_base,
                   int n_i, void* stream) {
  REQUIRE(planes && num && out, "bzpf_opm_outer: NULL pointer");
  REQUIRE(dt_ok(out_dt), "bzpf_opm_outer: bad dtype");
  REQUIRE(reinterpret_cast<uintptr_t>(planes) % 16 == 0, "bzpf_opm_outer: planes must be 16-byte aligned");
  REQUIRE(n_seq >= 1 && n_seq <= 16 * 65535 && N >= 1 && (int64_t)N * 6144 <= INT32_MAX && i_base >= 0 &&
              n_i >= 1 && i_base + n_i <= N,
          "bzpf_opm_outer: bad sizes (n_seq=%d N=%d i_base=%d n_i=%d)", n_seq, N, i_base, n_i);
  return done(bzpf::launch_opm_outer(planes, num, out, out_dt, n_seq, N, i_base, n_i, S(stream)), "bzpf_opm_outer");
}

int bzpf_transition64_f16(float* x, const float* ln_w, const float* ln_b, float eps, const void* w12, const void* w3,
                          int64_t rows, int hidden, void* stream) {
  REQUIRE(x && ln_w && ln_b && w12 && w3, "bzpf_transition64_f16: NULL pointer");
  REQUIRE(hidden >= 64 && hidden % 64 == 0 && hidden <= 384,
          "bzpf_transition64_f16: need hidden a multiple of 64, at most 384 (hidden=%d)", hidden);
  REQUIRE(reinterpret_cast<uintptr_t>(x) % 16 == 0 && reinterpret_cast<uintptr_t>(ln_w) % 16 == 0 &&
              reinterpret_cast<uintptr_t>(ln_b) % 16 == 0,
          "bzpf_transition64_f16: x, ln_w and ln_b must be 16-byte aligned");
  REQUIRE(rows >= 0, "bzpf_transition64_f16: rows < 0");
  if (rows == 0) return BZPF_OK;
  return done(bzpf::launch_transition64_f16(x, ln_w, ln_b, eps, w12, w3, rows, hidden, S(stream)),
              "bzpf_transition64_f16");
}

int bzpf_ln_linear_f32(const float* x, const float* ln_w, const float* ln_b, float eps, const float* w, float* y,
                       int64_t rows, int K, int M, void* stream) {
  REQUIRE(x && ln_w && ln_b && w && y, "bzpf_ln_linear_f32: NULL pointer");
  REQUIRE(K == 64 && M >= 256 && M % 256 == 0, "bzpf_ln_linear_f32: need K = 64 and M a multiple of 256 (K=%d M=%d)",
          K, M);
  REQUIRE(reinterpret_cast<uintptr_t>(x) % 16 == 0 && reinterpret_cast<uintptr_t>(w) % 16 == 0 &&
              reinterpret_cast<uintptr_t>(ln_w) % 16 == 0 && reinterpret_cast<uintptr_t>(ln_b) % 16 == 0,
          "bzpf_ln_linear_f32: x, w, ln_w and ln_b must be 16-byte aligned");
  REQUIRE(rows >= 0, "bzpf_ln_linear_f32: rows < 0");
  if (rows == 0) return BZPF_OK;
  return done(bzpf::launch_ln_linear_x3(x, ln_w, ln_b, eps, w, y, rows, K, M, S(stream)), "bzpf_ln_linear_f32");
}

int bzpf_pwa_softmax(const float* logits, const float* pair_mask, float inf, float* w, int N, int64_t ldw, int H,
                     void* stream) {
  REQUIRE(logits && pair_mask && w, "bzpf_pwa_softmax: NULL pointer");
  REQUIRE(N >= 1 && H >= 1 && ldw >= N && ldw % 16 == 0, "bzpf_pwa_softmax: bad sizes (N=%d H=%d ldw=%lld)", N, H,
          (long long)ldw);
  return done(bzpf::launch_pwa_softmax(logits, pair_mask, inf, w, N, ldw, H, S(stream)), "bzpf_pwa_softmax");
}

int64_t bzpf_pwa_wsplit_bytes(int N, int64_t ldw, int H) {
  if (N < 1 || H < 1 || ldw < N || ldw % 16) return -1;
  return bzpf::pwa_wsplit_bytes(N, ldw, H);
}

int bzpf_pwa_wsplit(const float* w, int64_t ldw, void* wp, int N, int H, void* stream) {
  REQUIRE(w && wp, "bzpf_pwa_wsplit: NULL pointer");
  REQUIRE(reinterpret_cast<uintptr_t>(w) % 8 == 0 && reinterpret_cast<uintptr_t>(wp) % 16 == 0,
          "bzpf_pwa_wsplit: w must be 8-byte and wp 16-byte aligned");
  REQUIRE(N >= 1 && H >= 1 && H <= 65535 && ldw >= N && ldw % 16 == 0, "bzpf_pwa_wsplit: bad sizes (N=%d H=%d)", N,
          H);
  return done(bzpf::launch_pwa_wsplit(w, ldw, wp, N, H, S(stream)), "bzpf_pwa_wsplit");
}

int bzpf_pwa_avg(const void* wp, int64_t ldw, const float* v, int64_t ldv, const float* g, int64_t ldg, float* out,
                 int64_t ldo, int n_seq, int N, int H, void* stream) {
  REQUIRE(wp && v && g && out, "bzpf_pwa_avg: NULL pointer");
  REQUIRE(reinterpret_cast<uintptr_t>(wp) % 16 == 0 && reinterpret_cast<uintptr_t>(v) % 16 == 0 && ldv % 4 == 0,
          "bzpf_pwa_avg: wp and v must be 16-byte aligned and ldv a multiple of 4");
  REQUIRE(n_seq >= 1 && n_seq <= 4 * 65535 && N >= 1 && H >= 1 && H <= 65535 && ldw >= N && ldw % 16 == 0 &&
              ldv >= 32 * H && ldg >= 32 * H && ldo >= 32 * H,
          "bzpf_pwa_avg: bad sizes (n_seq=%d N=%d H=%d)", n_seq, N, H);
  return done(bzpf::launch_pwa_avg(wp, ldw, v, ldv, g, ldg, out, ldo, n_seq, N, H, S(stream)), "bzpf_pwa_avg");
}

int bzpf_pair_bias(const float* z, const float* ln_w, const float* ln_b, float eps, const void* w, void* out, int dt,
                   int64_t rows, int D, int H, void* stream) {
  REQUIRE_PTR(z);
  REQUIRE_PTR(w);
  REQUIRE(ln_w && ln_b && out, "bzpf_pair_bias: NULL pointer");
  REQUIRE(dt_ok(dt), "bzpf_pair_bias: bad dtype");
  REQUIRE(D == 128 && H >= 1 && H <= 16, "bzpf_pair_bias: need D=128, 1 <= H <= 16 (D=%d H=%d)", D, H);
  REQUIRE(rows >= 0, "bzpf_pair_bias: rows < 0");
  if (rows == 0) return BZPF_OK;
  return done(bzpf::launch_pair_bias(z, ln_w, ln_b, eps, w, out, dt, rows, H, S(stream)), "bzpf_pair_bias");
}

}  // extern "C"
