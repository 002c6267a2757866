/*
 * bzpf — MI355X (gfx950) kernels for the Boltz-2 Pairformer pair path, C ABI.
 *
 * Every entry point takes device pointers, plain sizes and a hipStream_t passed as `void*`, launches on that
 * stream and returns 0, or a negative status (BZPF_EINVAL for a rejected argument, BZPF_ELAUNCH for a launch
 * failure) with a message in bzpf_last_error(). Nothing here allocates or frees device memory and nothing
 * synchronises: the caller owns every buffer (inputs, outputs and intermediates) and the stream order.
 *
 * Storage types: BZPF_F32 (fp32) or BZPF_F16 (fp16 operands, fp32 accumulation / statistics / softmax). The pair
 * representation z is always fp32 [N, N, 128] row-major. Pointers are 16-byte aligned; D = c_z = 128 for the
 * pair kernels.
 *
 * Each entry point replaces a kernel wrapper of the reference (paths relative to the reference checkout,
 * jackryan225/boltz-mlx), which launched MSL source through mx.fast.metal_kernel (boltz_mlx/kernels.py:315-324).
 */
#ifndef BZPF_H
#define BZPF_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define BZPF_F32 0
#define BZPF_F16 1

#define BZPF_OK 0
#define BZPF_EINVAL (-1)
#define BZPF_ELAUNCH (-2)

/* Library version string. */
const char* bzpf_version(void);

/* Message of the last failing call on this host thread ("" when none). */
const char* bzpf_last_error(void);

/* Row pitch (elements) of the padded pair buffers (triangle-multiplication a|b and o, triangle-attention V^T and
 * bias): N rounded up to 64. */
int64_t bzpf_row_pitch(int64_t N);

/* Row LayerNorm over D channels (D % 64 == 0, D <= 1024): two-pass fp32 statistics, (x-mean)*rsqrt(var+eps)*w+b;
 * w / b may be NULL. Replaces kernels.layer_norm (boltz_mlx/kernels.py:482-507) and LayerNorm.__call__/.f16
 * (boltz_mlx/layers/norm.py:9-17). */
int bzpf_layernorm(const void* x, int x_dt, const float* w, const float* b, float eps, void* y, int y_dt,
                   int64_t rows, int D, void* stream);

/* *count += the number of inf / nan among the n elements of x (fp32 or fp16; device int counter, no host sync): the
 * fp16 overflow guard's check of the residual streams. Replaces kernels.guard_residual / guard_take
 * (boltz_mlx/kernels.py:1262-1282) as used per recycle in boltz_mlx/model.py:176-193. */
int bzpf_count_nonfinite(const void* x, int dt, int64_t n, int* count, void* stream);

/* z[r] += y[trans_y ? T(r) : r] * y_scale over the N*N rows of z [N, N, D] (T swaps the two token axes); then,
 * when ln != NULL, ln[trans_out ? T(r) : r] = LN(z[r]). Replaces kernels.add_ln (boltz_mlx/kernels.py:1448-1480)
 * and kernels.radd (1305-1310). */
int bzpf_add_ln(float* z, const void* y, int y_dt, float y_scale, int trans_y, const float* w, const float* b,
                float eps, void* ln, int ln_dt, int trans_out, int64_t N, int D, void* stream);

/* Triangle-multiplication projection: for c < 2D and the position (i, k) (incoming: (k, i)),
 *   ab[c][i][k] = (xn.W[c]) * sigmoid(xn.W[2D + c]) * pair_mask * scale,  k < N;   ab[c][i][k] = 0 for N <= k < ld.
 * xn [N*N, D] (dt), W = [p_in.weight; g_in.weight] [4D, D] (dt), pair_mask [N, N] fp32, ab [2D][N][ld] (dt),
 * ld = bzpf_row_pitch(N). scale = 1 in fp32 mode, 2^-K in fp16 mode. Replaces the projection of
 * TriangleMultiplication._fast_b1 / _f16_contract (boltz_mlx/layers/triangular_mult.py:67-88, 143-170) and
 * kernels_nax2.trimul_proj_nax (boltz_mlx/kernels_nax2.py:202-304). */
int bzpf_trimul_proj(const void* xn, const void* w_pg, const float* pair_mask, float scale, int incoming, void* ab,
                     int dt, int64_t N, int64_t ld, int D, void* stream);

/* Per-channel contraction o[c][i][j] = sum_k ab[c][i][k] * ab[D + c][j][k] for c < D, o [D][N][ld] (dt; columns
 * j >= N are not written). k_len: when 0 < k_len < N, the caller guarantees that columns k >= k_len of ab are zero
 * (bzpf_trimul_proj writes zeros where the pair mask is zero, so k_len = 1 + the last token whose mask column
 * (outgoing) or row (incoming) is not all zero), and the sum stops at k_len rounded up to 64: the same result bit
 * for bit, without the trailing padded tokens' work. 0 (or >= N): every k. Replaces the mx.matmul contraction
 * (boltz_mlx/layers/triangular_mult.py:90-93, 172-175) and kernels_nax2.trimul_contract_nax
 * (boltz_mlx/kernels_nax2.py:315-407). */
int bzpf_trimul_contract(const void* ab, void* o, int dt, int64_t N, int64_t ld, int D, int64_t k_len, void* stream);

/* Triangle-multiplication tail: at each position p = (i, j),
 *   y = (LN_out(o[:, i, j]; eps_out) . W_po^T) * sigmoid(xn[p] . W_go^T);  z[p] = (accumulate ? z[p] : 0) + y;
 *   and, when next_w != NULL, xn_next[p] = LN_next(z[p]).
 * Replaces the output half of TriangleMultiplication (boltz_mlx/layers/triangular_mult.py:98-118) and
 * kernels_nax3.trimul_tail_addln / trimul_tail3_addln (boltz_mlx/kernels_nax3.py:200-268, 357-393, 1061-1206). */
int bzpf_trimul_tail(const void* o, const float* norm_out_w, const float* norm_out_b, float eps_out,
                     const void* w_po, const void* xn, const void* w_go, float* z, int accumulate,
                     const float* next_w, const float* next_b, float next_eps, void* xn_next, int dt, int64_t N,
                     int64_t ld, int D, void* stream);

/* Triangle-attention projection of the LayerNorm output xn [N*N, D] with W = [linear_q; linear_k; linear_v;
 * linear_g; linear] ([4*H*C + H, D]) at the position p = i*N + j (trans: xn is read at (j, i), the ending node):
 *   qkg [3H][N*N][C]: q * q_scale (planes 0..H-1), k (H..2H-1), g (2H..3H-1);
 *   vt [H][N][C][ldk]: v transposed per row i (vt[h][i][c][j] = v at (i, j)); columns j >= N are not written;
 *   tri_bias: bias_scale * (linear at (j, k)) for head h, query j, key k, in the fragment-ordered layout the
 *     attention core reads: with x = 16*((k%64)/32) + 4*((k%32)/8) + k%4 and lane = 32*((k%8)/4) + j%32, element
 *     (h, j, k) is at ((h*NJ + j/32)*(ldk/64) + k/64)*2048 + 512*(x/8) + 8*lane + x%8 with NJ = ceil(N/32)
 *     (H*32*NJ*ldk elements); keys N <= k < ldk are set to 0.
 * ldk = bzpf_row_pitch(N). bzpf_triattn_core expects q_scale = log2(e)/sqrt(C) and bias_scale = log2(e) (logits
 * in base 2). Replaces the fused projection of TriangleAttention
 * (boltz_mlx/layers/triangular_attention/attention.py:49-69, 100-104) and kernels_nax3.pair_proj16
 * (boltz_mlx/kernels_nax3.py:538-700). */
int bzpf_triattn_proj(const void* xn, const void* w, int trans, float q_scale, float bias_scale, void* qkg, void* vt,
                      void* tri_bias, int dt, int64_t N, int64_t ldk, int D, int H, int C, void* stream);

/* Flash triangle-attention core over the projection's buffers: for row i, head h, query j,
 *   out[i][j][h*C + c] = sigmoid(g) * sum_k softmax2_k(q.k + inf*(mask[i*mask_si + k*mask_sk] - 1)*log2(e)
 *                                                      + tri_bias(h, j, k)) v[k][c]
 * with softmax2 the base-2 softmax (2^x normalised; equal to the reference's softmax of the natural-log logits
 * (q/sqrt(C)).k + inf*(mask-1) + linear, summed in that order). fp32 softmax and accumulation; out [N*N, H*C] (dt).
 * impl selects the kernel like the reference's impl argument: 0 = auto (MFMA for fp16 with C = 32, else VALU),
 * 1 = the VALU kernel, 2 = the MFMA kernel (fp16, C = 32). With inf >= 1e6 the MFMA kernel skips the key blocks
 * after a row's last unmasked key (found among the row's last 256 keys): their probabilities are exactly zero, so
 * the output is the same bit for bit. Replaces kernels.tri_attention_fused
 * (boltz_mlx/kernels.py:531-945, impl "scalar" / "mma") and kernels_nax.tri_attention_nax
 * (boltz_mlx/kernels_nax.py:323-558). */
int bzpf_triattn_core(const void* qkg, const void* vt, const void* tri_bias, const float* mask, int64_t mask_si,
                      int64_t mask_sk, float inf, void* out, int dt, int64_t N, int64_t ldk, int H, int C, int impl,
                      void* stream);

/* Output projection + residual + next LayerNorm: y = x[p] . W^T (x [N*N, D], W [D, D]) added to z at the position
 * p (trans: the transposed position, the ending node), then xn_next = LN_next(z) at that position when
 * next_w != NULL. Replaces kernels_nax3.linear_addln (boltz_mlx/kernels_nax3.py:176-198, 320-354) and the
 * linear_o + radd of the strict path (boltz_mlx/layers/triangular_attention/attention.py:72-77). */
int bzpf_linear_resid_ln(const void* x, const void* w, int trans, float* z, int accumulate, const float* next_w,
                         const float* next_b, float next_eps, void* xn_next, int dt, int64_t N, int D, void* stream);

/* Transition: z[r] = (accumulate ? z[r] : 0) + fc3(silu(xn[r].fc1^T) * (xn[r].fc2^T)) over `rows` rows of D = 128,
 * w12 = [fc1.weight; fc2.weight] [2*hidden, D], w3 = fc3.weight [D, hidden]; then xn_next = LN_next(z) when
 * next_w != NULL. Replaces kernels.transition_fused (boltz_mlx/kernels.py:1122-1155),
 * kernels_nax2.transition_nax (boltz_mlx/kernels_nax2.py:54-190) and kernels_nax3.transition_lnx / transition3
 * (boltz_mlx/kernels_nax3.py:713-827, 1381-1482). */
int bzpf_transition(const void* xn, const void* w12, const void* w3, float* z, int accumulate, const float* next_w,
                    const float* next_b, float next_eps, void* xn_next, int dt, int64_t rows, int D, int hidden,
                    void* stream);

/* bzpf_transition, then the s track's pair bias from the updated z: pb_out[h][r] = Linear(LN_pb(z[r]))[h] over the
 * same rows ([pb_heads][rows] in dt; pb_w [pb_heads, D] in dt, pb_lnw/pb_lnb fp32 [D], 1 <= pb_heads <= 16), as
 * bzpf_pair_bias computes it. In fp16 the transition's epilogue computes it from the row statistics it already has
 * (fp16 MFMA on the normalised row with gamma_pb folded into the weights), so z is not read again. Replaces the
 * reference's proj_z fusion into the pair transition epilogue (boltz_mlx/kernels_nax3.py:702-768). */
int bzpf_transition_pb(const void* xn, const void* w12, const void* w3, float* z, int accumulate, const float* next_w,
                       const float* next_b, float next_eps, void* xn_next, const void* pb_w, const float* pb_lnw,
                       const float* pb_lnb, float pb_eps, void* pb_out, int pb_heads, int dt, int64_t rows, int D,
                       int hidden, void* stream);

/* The ending-node attention's output stage and the pair transition in one pass (fp16 only, D = 128): for every pair
 * row r = (i, j) of z [N*N][128] fp32,
 *   z[r] += o[r'] . w_o^T,  r' = (j, i) when trans (the attention frame of the ending node), else r;
 *   xn = LN(z[r]) with ln_w / ln_b / ln_eps (the transition's own norm, fp16);
 *   z[r] += fc3(silu(xn . fc1^T) * (xn . fc2^T)),
 * then next LN and (pb_w != NULL) the s track's pair bias as in bzpf_transition_pb. Equals bzpf_linear_resid_ln
 * (accumulate = 1, next LN = the transition's norm) followed by bzpf_transition(_pb) bit for bit, without writing
 * and reading back the intermediate xn. Replaces the triangle attention's linear_o + residual
 * (f16_addln, boltz_mlx/layers/triangular_attention/attention.py:170-190) followed by the pair transition
 * (boltz_mlx/layers/transition.py:50-54; kernels_nax3.transition_lnx, boltz_mlx/kernels_nax3.py:713-827). */
int bzpf_attn_out_transition(const void* o, const void* w_o, int trans, const float* ln_w, const float* ln_b,
                             float ln_eps, const void* w12, const void* w3, float* z, const float* next_w,
                             const float* next_b, float next_eps, void* xn_next, const void* pb_w,
                             const float* pb_lnw, const float* pb_lnb, float pb_eps, void* pb_out, int pb_heads, int dt,
                             int64_t N, int D, int hidden, void* stream);

/* Linear layer y[r] = x[r] . W^T + bias (K % 8 == 0; bias may be NULL); accumulate != 0 adds into an fp32 y.
 * Replaces the nn.Linear / kernels.lin16 calls of the s track (boltz_mlx/layers/attentionv2.py:50-52, 70, 84;
 * boltz_mlx/kernels.py:1360-1370). */
int bzpf_linear(const void* x, const void* w, const float* bias, void* y, int dt, int y_dt, int64_t rows, int K,
                int M, int accumulate, void* stream);

/* The same layer written out of place onto a residual: y[r] = res[r] + x[r] . W^T + bias for fp32 y [rows, M] and
 * fp32 res rows of pitch ld_res (16-byte aligned, ld_res % 4 == 0; res may not overlap y), the same sums as copying
 * res into y and calling bzpf_linear with accumulate. The residual updates of the MSA block
 * (boltz_mlx/layers/msa.py: m + pair_weighted_averaging(m), z + outer_product_mean(m)) without copying the inputs. */
int bzpf_linear_residual(const void* x, const void* w, const float* bias, const float* res, int64_t ld_res, float* y,
                         int dt, int64_t rows, int K, int M, void* stream);

/* a[r][c] = silu(h[r][c]) * h[r][hidden + c]. Replaces the SwiGLU of Transition
 * (boltz_mlx/layers/transition.py:148-154; kernels.swiglu16, boltz_mlx/kernels.py:1378-1386). */
int bzpf_swiglu(const void* h, void* a, int dt, int64_t rows, int hidden, void* stream);

/* y[r][m] += sigmoid(gate[(r % gate_rows) * ld_gate + m]) * (x[r] . W[m] + bias[m]) with y fp32 (bias may be
 * NULL): a gated residual update. Replaces the diffusion transformer's a + sigmoid(output_projection(s)) * proj_o(..)
 * and a + sigmoid(output_projection(s)) * b_to_a(..) (boltz_mlx/modules/transformersv2.py:63-66, 96-99, 239, 261). */
int bzpf_linear_gated(const void* x, const void* w, const float* bias, const float* gate, int64_t ld_gate,
                      int64_t gate_rows, float* y, int dt, int64_t rows, int K, int M, void* stream);

/* a[r][c] = silu(h[r][c]) * h[r][hidden + c] * h[r][2 hidden + c] (rows of h: 3 hidden). Replaces the conditioned
 * transition's SwiGLU(swish_gate(a)) * a_to_b(a) with the GEMM rows ordered [gates; x; a_to_b]
 * (boltz_mlx/modules/transformersv2.py:15-18, 55-66, 254-261). */
int bzpf_swiglu3(const void* h, void* a, int dt, int64_t rows, int hidden, void* stream);

/* AdaLN: out[r][c] = sigmoid(scale[q][c]) * LN(a[r])[c] + shift[q][c] with q = r % cond_rows (conditioning rows of
 * pitch ld_cond, fp32, pre-sigmoid scale), LN without affine over D channels, a fp32. Replaces AdaLN.__call__ and
 * the fast path's attn_scale * LN(a) + attn_shift (boltz_mlx/modules/transformersv2.py:27-41, 218, 252). */
int bzpf_adaln(const float* a, const float* scale, const float* shift, int64_t ld_cond, int64_t cond_rows, float eps,
               void* out, int out_dt, int64_t rows, int D, void* stream);

/* Sequence attention with pair bias: for head h and query j,
 *   out[j][h*hd + c] = sigmoid(g[j][h*hd + c]) * sum_k softmax_k(q.k/sqrt(hd) + bias[h][j][k]
 *                                                                 + (1 - mask[k]) * (-inf)) v[k][h*hd + c]
 * q/k/v/g rows of pitch ld_in, out rows of pitch ld_out; q/k/v/g/out are of type dt, the bias of type bias_dt (the
 * reference's f16 mode adds an fp16 pair bias to fp32 logits: dt = fp32, bias_dt = fp16). Replaces the attention
 * core of AttentionPairBias (boltz_mlx/layers/attentionv2.py:70-83). */
int bzpf_seq_attention(const void* q, const void* k, const void* v, const void* g, int64_t ld_in, const void* bias,
                       const float* mask, float inf, void* out, int64_t ld_out, int dt, int bias_dt, int64_t N, int H,
                       int hd, void* stream);

/* bzpf_seq_attention over n_samples samples in one call: sample i reads q/k/v/g rows from q + i*s_in (elements),
 * the mask row mask + i*s_mask, the bias bias + (i / mult)*s_bias (mult consecutive samples share one [H, N, N]
 * bias) and writes out + i*s_out. Replaces the batched attention of the diffusion transformer's AttentionPairBias
 * over B * multiplicity samples (boltz_mlx/modules/transformersv2.py:218-239, boltz_mlx/layers/attentionv2.py:59-83). */
int bzpf_seq_attention_batched(const void* q, const void* k, const void* v, const void* g, int64_t ld_in,
                               int64_t s_in, const void* bias, int64_t s_bias, int mult, const float* mask,
                               int64_t s_mask, float inf, void* out, int64_t ld_out, int64_t s_out, int dt,
                               int bias_dt, int n_samples, int64_t N, int H, int hd, void* stream);

/* Pair updates at channel counts other than 128 (the template stack's c_z = 64): the projections run as bzpf_linear
 * GEMMs over xn [N*N, D] and these three calls move their outputs into the layouts bzpf_trimul_contract and
 * bzpf_triattn_core read (the fused bzpf_trimul_proj / bzpf_triattn_proj / bzpf_trimul_tail need D = 128).
 *
 * bzpf_trimul_pack: P [N*N, 4D] = xn [p_in; g_in]^T -> ab [2D][N][ld] with
 *   ab[c][i][k] = P[p][c] * sigmoid(P[p][2D + c]) * mask[p] * scale, p = i*N + k (outgoing) or k*N + i (incoming),
 * zeros for N <= k < ld; mask fp32 [N, N], ld = bzpf_row_pitch(N), D <= 4096. Replaces the projection of the
 * reference's TriangleMultiplication (boltz_mlx/layers/triangular_mult.py:40-65, 143-170). */
int bzpf_trimul_pack(const void* P, const float* mask, float scale, int incoming, void* ab, int dt, int64_t N,
                     int64_t ld, int D, void* stream);

/* bzpf_channels_to_rows: out[i*N + j][c] = o[c][i][j] for o [D][N][ld] (the contraction output) -> out [N*N, D]
 * (dtypes independent), the operand of norm_out (boltz_mlx/layers/triangular_mult.py:93-98). D <= 252. */
int bzpf_channels_to_rows(const void* o, int o_dt, void* out, int out_dt, int64_t N, int64_t ld, int D,
                          void* stream);

/* bzpf_triattn_pack: P [N*N, 4*H*C + H] = xn [linear_q; linear_k; linear_v; linear_g; linear]^T -> the qkg, vt and
 * fragment-ordered tri_bias buffers of bzpf_triattn_proj (same layouts, q * q_scale, bias * bias_scale), P read at
 * (j, i) when trans (the ending node). tri_bias rows of padded queries (N <= j < 32*ceil(N/32)) are not written:
 * the caller zeroes the buffer. H*C + H <= 252. Replaces the projection of the reference's TriangleAttention
 * (boltz_mlx/layers/triangular_attention/attention.py:49-69, 100-104) at any c_in. */
int bzpf_triattn_pack(const void* P, int trans, float q_scale, float bias_scale, void* qkg, void* vt, void* tri_bias,
                      int dt, int64_t N, int64_t ldk, int H, int C, void* stream);

/* The conditioned transition's feed-forward GEMM with its gated product fused (fp16 only):
 *   u[r][c] = silu(x[r] . Wg[c]) * (x[r] . Wx[c]) * (x[r] . Wab[c])   for r < rows, c < H,
 * x fp16 [rows, K] (K % 64 == 0), u fp16 [rows, H] (H % 32 == 0), fp32 accumulation; w fp16 [3H, K] in 96-row groups
 * [Wg[32 q .. 32 q + 31]; Wx[same]; Wab[same]] for q < H / 32 (Wg = the second half of swish_gate.0.weight, Wx its
 * first half, Wab = a_to_b.weight). Replaces swish_gate + SwiGLU + a_to_b of ConditionedTransitionBlock
 * (boltz_mlx/modules/transformersv2.py:44-66, kernels_nax3.py:447-700): bzpf_linear + bzpf_swiglu3 without the
 * [rows, 3H] intermediate. */
int bzpf_linear_swiglu3(const void* x, const void* w, void* u, int64_t rows, int K, int H, void* stream);

/* The same for Transition's SwiGLU: u[r][c] = silu(x[r] . W1[c]) * (x[r] . W2[c]) with w fp16 [2H, K] in 64-row
 * groups [W1[32 q .. 32 q + 31]; W2[same]] (W1 = fc1.weight, W2 = fc2.weight). Replaces fc1 / fc2 and the SwiGLU of
 * Transition (boltz_mlx/layers/transition.py:27-92): bzpf_linear + bzpf_swiglu without the [rows, 2H]
 * intermediate. */
int bzpf_linear_swiglu(const void* x, const void* w, void* u, int64_t rows, int K, int H, void* stream);

/* Outer-product-mean operands, masked and split for bzpf_opm_outer: for MSA rows s < n_seq and tokens n < N
 * (fp32 ab [n_seq, N, ld_ab]: a = ab[.., 0:32], b = ab[.., 32:64], unmasked; mask fp32 [n_seq, N]) the products
 * x = mask[s][n] * ab[s][n][ch] as three bf16 parts x = x1 + x2 + x3 (exact; x1 = bf16(x), x2 = bf16(x - x1)).
 * planes: 16-byte aligned, ceil(n_seq / 16) * N * 6144 bytes; 1 KB chunk (g, n, p, h) at byte
 * ((g * N + n) * 6 + 2 * p + h) * 1024 holds part p + 1 of channels 32 h .. 32 h + 31 of token n over MSA rows
 * 16 g .. 16 g + 15, as 32 rows (channel) of 16 bf16 (MSA row), zeros past n_seq. The masking of a and b in
 * kernels_msa.opm_outer's operand staging (boltz_mlx/kernels_msa.py:292-343,
 * boltz_mlx/layers/outer_product_mean.py:37-45). */
int bzpf_opm_split(const float* ab, int64_t ld_ab, const float* mask, void* planes, int n_seq, int N, void* stream);

/* The same planes from the MSA itself: x = mask[s][n] * (LN(m[s][n]; ln_w, ln_b, eps) . W_ab[ch]) for m fp32
 * [n_seq, N, 64], W_ab fp32 [64, 64] = [proj_a.weight; proj_b.weight], mask fp32 [n_seq, N], in one kernel (the
 * LayerNorm of bzpf_layernorm; each product the six bf16 part products of the three-part split, fp32 accuracy).
 * Replaces norm + proj_a / proj_b + the masking of OuterProductMean (boltz_mlx/layers/outer_product_mean.py:37-45,
 * boltz_mlx/kernels_msa.py:292-343): bzpf_layernorm + bzpf_linear + bzpf_opm_split without the intermediates. */
int bzpf_opm_ln_split(const float* m, const float* ln_w, const float* ln_b, float eps, const float* w_ab,
                      const float* mask, void* planes, int n_seq, int N, void* stream);

/* Outer-product-mean outer sum over the planes of bzpf_opm_split: for i_base <= i < i_base + n_i and j < N,
 *   out[(i - i_base) * N + j][c * 32 + d] = sum_s mask[s][i] mask[s][j] a[s][i][c] b[s][j][d] / max(num[i][j], 1),
 * num fp32 [N, N] = mask^T mask (the pair counts; one bzpf_linear of the transposed mask with itself, as the
 * reference's num input); out fp16 or fp32 [n_i * N, 1024]. Each product is the six bf16 part products x_a y_b with
 * a + b <= 4, accumulated in fp32 (fp32 accuracy). Replaces kernels_msa.opm_outer and the module path's outer sum
 * (boltz_mlx/kernels_msa.py:292-343, boltz_mlx/layers/outer_product_mean.py:37-45). */
int bzpf_opm_outer(const void* planes, const float* num, void* out, int out_dt, int n_seq, int N, int i_base, int n_i,
                   void* stream);

/* The 64-channel Transition in fp16, in place, in one kernel: x += fc3(silu(xn fc1^T) * (xn fc2^T)) with
 * xn = fp16(LN(x; ln_w, ln_b, eps)), for x fp32 [rows, 64], w12 fp16 [2 hidden, 64] = [fc1; fc2], w3 fp16
 * [64, hidden] (hidden a multiple of 64, at most 384); fp32 accumulation, the SwiGLU product rounded to fp16 as the
 * fc3 operand. Replaces Transition at 64 channels (boltz_mlx/layers/transition.py:27-92; the MSA track's
 * transition): bzpf_layernorm + bzpf_linear_swiglu + bzpf_linear without the [rows, hidden] intermediate. */
int bzpf_transition64_f16(float* x, const float* ln_w, const float* ln_b, float eps, const void* w12, const void* w3,
                          int64_t rows, int hidden, void* stream);

/* The MSA track's LayerNorm + fp32 Linear in one kernel: y[r][m] = LN(x[r]; ln_w, ln_b, eps) . W[m] for x fp32
 * [rows, K = 64], W fp32 [M, 64] (M a multiple of 256), y fp32 [rows, M]. The LayerNorm is bzpf_layernorm's arithmetic;
 * each product is the six bf16 part products of the three-part split (fp32 accuracy). Replaces norm_m + proj_m |
 * proj_g of PairWeightedAveraging (boltz_mlx/layers/pair_averaging.py:36-41): bzpf_layernorm + bzpf_linear without
 * the [rows, 64] intermediate. */
int bzpf_ln_linear_f32(const float* x, const float* ln_w, const float* ln_b, float eps, const float* w, float* y,
                       int64_t rows, int K, int M, void* stream);

/* Pair-weighted-averaging weights: w[h][i][j] = softmax_j(logits[h][i][j] + (1 - pair_mask[i][j]) * -inf) for
 * logits fp32 [H, N, N], pair_mask fp32 [N, N]; w fp32 [H, N, ldw] with zeros for N <= j < ldw (ldw a multiple of
 * 16 and >= N). Replaces the softmax of kernels_msa.pwa_weights (boltz_mlx/kernels_msa.py:461-500,
 * boltz_mlx/layers/pair_averaging.py:43-49); the logits are bzpf_pair_bias of z with the fp32 proj_z weight. */
int bzpf_pwa_softmax(const float* logits, const float* pair_mask, float inf, float* w, int N, int64_t ldw, int H,
                     void* stream);

/* The weights of bzpf_pwa_softmax (w fp32 [H, N, ldw]) as three exact bf16 parts w = w1 + w2 + w3 for
 * bzpf_pwa_avg: wp (16-byte aligned, bzpf_pwa_wsplit_bytes(N, ldw, H) bytes) holds 1 KB chunk (h, ib, jg, p) at byte
 * (((h * ceil(N / 32) + ib) * G + jg) * 3 + p) * 1024 (G = ldw / 16 rounded up to even): part p + 1 of w[h][i][j]
 * for i = 32 ib .. + 31, j = 16 jg .. + 15 (zeros past N and past ldw), as 32 rows of 16 bf16. The weights' operand staging of kernels_msa.pwa_avg
 * (boltz_mlx/kernels_msa.py:620-653). bzpf_pwa_wsplit_bytes returns -1 for bad sizes. */
int64_t bzpf_pwa_wsplit_bytes(int N, int64_t ldw, int H);
int bzpf_pwa_wsplit(const float* w, int64_t ldw, void* wp, int N, int H, void* stream);

/* Pair-weighted average with its gate: out[s][i][h*32 + d] = sigmoid(g[s][i][h*32 + d]) *
 * sum_j w[h][i][j] v[s][j][h*32 + d] for the split weights wp of bzpf_pwa_wsplit (ldw as given there) and v, g, out
 * fp32 rows (s, i) of pitch ldv / ldg / ldo. Each product is the six bf16 part products w_a v_b with a + b <= 4,
 * accumulated in fp32 (fp32 accuracy). Replaces kernels_msa.pwa_avg (boltz_mlx/kernels_msa.py:620-653,
 * boltz_mlx/layers/pair_averaging.py:50-57). */
int bzpf_pwa_avg(const void* wp, int64_t ldw, const float* v, int64_t ldv, const float* g, int64_t ldg, float* out,
                 int64_t ldo, int n_seq, int N, int H, void* stream);

/* Pair bias out[h][r] = LN(z[r]; ln_w, ln_b, eps) . W[h] for r < rows (z fp32 [rows, D = 128], W [H, D], H <= 16).
 * Replaces proj_z of AttentionPairBias (boltz_mlx/layers/attentionv2.py:37-39, 57-66) and the pair-bias epilogue of
 * kernels_nax3.transition_lnx (boltz_mlx/kernels_nax3.py:713-768). */
int bzpf_pair_bias(const float* z, const float* ln_w, const float* ln_b, float eps, const void* w, void* out, int dt,
                   int64_t rows, int D, int H, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* BZPF_H */
