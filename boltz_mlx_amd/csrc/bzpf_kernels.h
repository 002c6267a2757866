// Internal launchers (host side) behind the C-ABI in bzpf_api.hip. All take device pointers and launch on `st`.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace bzpf {

enum { DT_F32 = 0, DT_F16 = 1 };

hipError_t launch_layernorm(const void* x, int x_dt, const float* w, const float* b, float eps, void* y, int y_dt,
                            int64_t rows, int D, hipStream_t st);
hipError_t launch_add_ln(float* z, const void* y, int y_dt, float scale, int trans_y, const float* w, const float* b,
                         float eps, void* ln, int ln_dt, int trans_out, int64_t N, int D, hipStream_t st);
hipError_t launch_count_nonfinite(const void* x, int dt, int64_t n, int* count, hipStream_t st);

hipError_t launch_trimul_proj(const void* xn, const void* w, const float* mask, float scale, int incoming, void* ab,
                              int dt, int64_t N, int64_t ld, hipStream_t st);
hipError_t launch_trimul_contract(const void* ab, void* o, int dt, int64_t N, int64_t ld, int64_t k_len, int D,
                                  hipStream_t st);
hipError_t launch_trimul_tail(const void* o, const float* now, const float* nob, float eps_out, const void* w_po,
                              const void* xn, const void* w_go, float* z, int accumulate, const float* lnw,
                              const float* lnb, float eps_next, void* xn_next, int dt, int64_t N, int64_t ld,
                              hipStream_t st);

hipError_t launch_triattn_proj(const void* xn, const void* w, int trans, float q_scale, float b_scale, void* qkg,
                               void* vt, void* tb, int dt, int64_t N, int64_t ldk, int H, int C, hipStream_t st);
hipError_t launch_triattn_core(const void* qkg, const void* vt, const void* tb, const float* mask, int64_t mask_si,
                               int64_t mask_sk, float inf, void* out, int dt, int64_t N, int64_t ldk, int H, int C,
                               int impl, hipStream_t st);
hipError_t launch_triattn_core_f16_mfma(const void* qkg, const void* vt, const void* tb, const float* mask,
                                        int64_t mask_si, int64_t mask_sk, float inf, void* out, int64_t N,
                                        int64_t ldk, int H, int C, hipStream_t st);
hipError_t launch_triattn_core_simple(const void* qkg, const void* vt, const void* tb, const float* mask,
                                      int64_t mask_si, int64_t mask_sk, float inf, void* out, int dt, int64_t N,
                                      int64_t ldk, int H, int C, hipStream_t st);
hipError_t launch_linear_resid_ln(const void* x, const void* w, int trans, float* z, int accumulate,
                                  const float* lnw, const float* lnb, float eps, void* xn_next, int dt, int64_t N,
                                  hipStream_t st);
hipError_t launch_transition(const void* xn, const void* w12, const void* w3, float* z, int accumulate,
                             const float* lnw, const float* lnb, float eps, void* xn_next, int dt, int64_t rows,
                             int hidden, hipStream_t st);
hipError_t launch_transition_pb(const void* xn, const void* w12, const void* w3, float* z, int accumulate,
                                const float* lnw, const float* lnb, float eps, void* xn_next, const void* pb_w,
                                const float* pb_lnw, const float* pb_lnb, float pb_eps, void* pb_out, int pb_heads,
                                int dt, int64_t rows, int hidden, hipStream_t st);
hipError_t launch_attn_out_transition(const void* o, const void* w_o, int trans, const float* ln_w, const float* ln_b,
                                      float ln_eps, const void* w12, const void* w3, float* z, const float* next_w,
                                      const float* next_b, float next_eps, void* xn_next, const void* pb_w,
                                      const float* pb_lnw, const float* pb_lnb, float pb_eps, void* pb_out,
                                      int pb_heads, int64_t N, int hidden, hipStream_t st);

hipError_t launch_linear(const void* x, const void* w, const float* bias, void* y, int dt, int y_dt, int64_t rows,
                         int K, int M, int epi, hipStream_t st);
// Tiled MFMA GEMM (64- or 128-row tiles; fp16 or fp32 operands) behind launch_linear / launch_linear_gated when K
// is a multiple of 128 bytes, M % 4 == 0 and the operands are 16-byte aligned (gemm_nt_ok)
bool gemm_nt_ok(int x_dt, const void* x, const void* w, const float* bias, const void* y, int64_t R, int K, int M,
                const float* gate, int64_t ld_gate);
hipError_t launch_gemm_nt(const void* x, const void* w, const float* bias, void* y, int x_dt, int y_dt, int64_t R,
                          int K, int M, int epi, const float* gate, int64_t ld_gate, int64_t gate_rows,
                          hipStream_t st);
hipError_t launch_gemm_swiglu_f16(const void* x, const void* w, void* u, int64_t R, int K, int H, int np,
                                  hipStream_t st);
hipError_t launch_swiglu(const void* h, void* a, int dt, int64_t R, int H, hipStream_t st);
hipError_t launch_swiglu3(const void* h, void* a, int dt, int64_t R, int H, hipStream_t st);
hipError_t launch_linear_gated(const void* x, const void* w, const float* bias, const float* gate, int64_t ld_gate,
                               int64_t gate_rows, float* y, int dt, int64_t rows, int K, int M, hipStream_t st);
hipError_t launch_adaln(const float* a, const float* scale, const float* shift, int64_t ldc, int64_t cond_rows,
                        float eps, void* out, int out_dt, int64_t R, int D, hipStream_t st);
hipError_t launch_seq_attention_f16_mfma(const void* q, const void* k, const void* v, const void* g, int64_t ld_in,
                                         int64_t s_in, const void* bias, int64_t s_bias, int mult, const float* mask,
                                         int64_t s_mask, float inf, void* out, int64_t ld_out, int64_t s_out,
                                         int S, int64_t N, int H, int hd, hipStream_t st);
hipError_t launch_seq_attention_f32_mfma(const void* q, const void* k, const void* v, const void* g, int64_t ld_in,
                                         int64_t s_in, const void* bias, int64_t s_bias, int mult, const float* mask,
                                         int64_t s_mask, float inf, void* out, int64_t ld_out, int64_t s_out,
                                         int bias_dt, int S, int64_t N, int H, int hd, hipStream_t st);
hipError_t launch_seq_attention(const void* q, const void* k, const void* v, const void* g, int64_t ld_in,
                                int64_t s_in, const void* bias, int64_t s_bias, int mult, const float* mask,
                                int64_t s_mask, float inf, void* out, int64_t ld_out, int64_t s_out, int dt,
                                int bias_dt, int S, int64_t N, int H, int hd, hipStream_t st);
hipError_t launch_opm_split(const float* ab, int64_t ld_ab, const float* mask, void* planes, int S, int N,
                            hipStream_t st);
hipError_t launch_opm_outer(const void* planes, const float* num, void* out, int out_dt, int S, int N, int i_base,
                            int n_i, hipStream_t st);
hipError_t launch_opm_ln_split(const float* m, const float* lnw, const float* lnb, float eps, const float* w_ab,
                               const float* mask, void* planes, int S, int N, hipStream_t st);
hipError_t launch_transition64_f16(float* x, const float* lnw, const float* lnb, float eps, const void* w12,
                                   const void* w3, int64_t R, int H, hipStream_t st);
hipError_t launch_ln_linear_x3(const float* x, const float* lnw, const float* lnb, float eps, const float* w, float* y,
                               int64_t R, int K, int M, hipStream_t st);
hipError_t launch_pwa_softmax(const float* logits, const float* pm, float inf, float* w, int N, int64_t ldw, int H,
                              hipStream_t st);
int64_t pwa_wsplit_bytes(int N, int64_t ldw, int H);
hipError_t launch_pwa_wsplit(const float* w, int64_t ldw, void* wp, int N, int H, hipStream_t st);
hipError_t launch_pwa_avg(const void* wp, int64_t ldw, const float* v, int64_t ldv, const float* g, int64_t ldg,
                          float* out, int64_t ldo, int S, int N, int H, hipStream_t st);
hipError_t launch_trimul_pack(const void* P, const float* mask, float scale, int incoming, void* ab, int dt,
                              int64_t N, int64_t ld, int D, hipStream_t st);
hipError_t launch_channels_to_rows(const void* o, int o_dt, void* out, int out_dt, int64_t N, int64_t ld, int D,
                                   hipStream_t st);
hipError_t launch_triattn_pack(const void* P, int trans, float q_scale, float b_scale, void* qkg, void* vt, void* tb,
                               int dt, int64_t N, int64_t ldk, int H, int C, hipStream_t st);
hipError_t launch_pair_bias(const float* z, const float* lnw, const float* lnb, float eps, const void* w, void* out,
                            int dt, int64_t rows, int H, hipStream_t st);

}  // namespace bzpf
