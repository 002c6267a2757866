// Attention cores on VALU: the triangle-attention reference kernel (any storage type and head width; the fp16 MFMA
// kernel is in bzpf_triattn_mfma.hip) and the sequence-track attention with pair bias. The projection and the
// output projection of triangle attention are in bzpf_pair_gemm.hip.
// Reference behaviour: boltz_mlx/layers/triangular_attention/attention.py:27-93 (fp32), 95-190 (f16),
// primitives.py:40-75 (q scaled before q.k; logits + mask_bias + tri_bias), kernels.py:538-600 (summation order
// (qk + mask_bias) + tri_bias), kernels_nax3.py:176-198 (linear_o + residual + next LN, transposed read of z).
#include "bzpf_common.h"
#include "bzpf_kernels.h"

namespace bzpf {

// ---------------------------------------------------------------- triangle attention core (reference VALU kernel)
// One thread per query j; a 64-thread workgroup owns (row i, head h, 64 queries). K, V^T and the [64 x TK] bias
// tile are staged TK keys at a time in LDS with coalesced loads. Logits are in base 2: q carries log2(e)/sqrt(C)
// and the bias log2(e) (both applied by the projection), the key-mask bias is inf*(m-1)*log2(e); the order is the
// reference's ((q.k) + mask_bias) + tri_bias and p = 2^(x - max).
template <typename T, int C>
__global__ __launch_bounds__(64) void triattn_core_valu(const T* __restrict__ qkg, const T* __restrict__ vt,
                                                       const T* __restrict__ tb, const float* __restrict__ mask,
                                                       int64_t mask_si, int64_t mask_sk, float inf,
                                                       T* __restrict__ out, int64_t N, int64_t ldk, int H) {
  constexpr int TK = 32;
  constexpr float LOG2E = 1.4426950408889634f;
  __shared__ float Ks[TK][C + 1];
  __shared__ float Vs[TK][C + 1];
  __shared__ float Bs[64][TK + 1];
  __shared__ float Mk[TK];
  const int t = threadIdx.x;
  const int64_t NN = N * N;
  const int64_t j = (int64_t)blockIdx.x * 64 + t, j0 = (int64_t)blockIdx.x * 64;
  const int64_t h = blockIdx.y, i = blockIdx.z;
  const bool valid = j < N;
  const T* qb = qkg + (h * NN + i * N) * C;
  const T* kb = qkg + ((H + h) * NN + i * N) * C;
  const T* gb = qkg + ((2 * H + h) * NN + i * N) * C;
  const T* vb = vt + (h * N + i) * C * ldk;
  float q[C], acc[C];
#pragma unroll
  for (int d = 0; d < C; d++) {
    q[d] = valid ? to_f(qb[j * C + d]) : 0.f;
    acc[d] = 0.f;
  }
  float m = -INFINITY, lsum = 0.f;
  for (int64_t k0 = 0; k0 < N; k0 += TK) {
    __syncthreads();
    for (int e = t; e < TK * C; e += 64) {
      const int kk = e / C, d = e - kk * C;
      Ks[kk][d] = k0 + kk < N ? to_f(kb[(k0 + kk) * C + d]) : 0.f;
      const int d2 = e / TK, k2 = e - d2 * TK;
      Vs[k2][d2] = k0 + k2 < N ? to_f(vb[d2 * ldk + k0 + k2]) : 0.f;
    }
    for (int e = t; e < 64 * TK; e += 64) {
      const int qq = e / TK, kk = e - qq * TK;
      Bs[qq][kk] = (j0 + qq < N && k0 + kk < N) ? to_f(tb[tb_offset(h, j0 + qq, k0 + kk, N, ldk)]) : 0.f;
    }
    if (t < TK) Mk[t] = k0 + t < N ? inf * (mask[i * mask_si + (k0 + t) * mask_sk] - 1.0f) * LOG2E : 0.f;
    __syncthreads();
    const int kend = (int)((N - k0) < TK ? (N - k0) : TK);
    for (int kk = 0; kk < kend; kk++) {
      float s = 0.f;
#pragma unroll
      for (int d = 0; d < C; d++) s += q[d] * Ks[kk][d];
      s += Mk[kk];
      s += Bs[t][kk];
      const float mn = fmaxf(m, s);
      const float corr = exp2f(m - mn);
      const float p = exp2f(s - mn);
      lsum = lsum * corr + p;
#pragma unroll
      for (int d = 0; d < C; d++) acc[d] = acc[d] * corr + p * Vs[kk][d];
      m = mn;
    }
  }
  if (!valid) return;
  const float inv = 1.0f / lsum;
  T* ob = out + (i * N + j) * (int64_t)(H * C) + h * C;
#pragma unroll
  for (int d = 0; d < C; d++) ob[d] = from_f<T>(acc[d] * inv * sigmoidf_(to_f(gb[j * C + d])));
}

// ---------------------------------------------------------------- sequence attention (s track, VALU kernel)
// AttentionPairBias core (attentionv2.py:76-83): for head h and query j,
//   out[j][h*hd + d] = sigmoid(g[j][h*hd + d]) * sum_k softmax_k(q.k * scale + bias[h][j][k] + (1 - mask[k]) * -inf) v
// A 256-thread workgroup owns (head h, 16 queries); the 16 threads of a query split the keys (key = 16 * t + lane)
// with an online softmax each, and merge their (max, sum, accumulator) states with shuffles at the end. K, V and
// the [16 x 64] bias tile are staged 64 keys at a time in LDS. The bias type TB may differ from T (fp32 logits with
// an fp16 pair bias, the reference's f16-mode s track).
template <typename T, typename TB, int HD>
__global__ __launch_bounds__(256) void seq_attn_kernel(const T* __restrict__ q, const T* __restrict__ k,
                                                       const T* __restrict__ v, const T* __restrict__ g,
                                                       int64_t ld_in, const TB* __restrict__ bias,
                                                       const float* __restrict__ mask, float inf,
                                                       T* __restrict__ out, int64_t ld_out, int64_t N, float scale) {
  constexpr int TK = 64;
  __shared__ float Ks[TK][HD + 1];
  __shared__ float Vs[TK][HD + 1];
  __shared__ float Bs[16][TK + 1];
  __shared__ float Mk[TK];
  const int t = threadIdx.x, qi = t >> 4, kl = t & 15;
  const int h = blockIdx.y;
  const int64_t j0 = (int64_t)blockIdx.x * 16, j = j0 + qi;
  const bool valid = j < N;
  const int64_t jc = valid ? j : N - 1;
  float qv[HD], acc[HD];
#pragma unroll
  for (int d = 0; d < HD; d++) {
    qv[d] = to_f(q[jc * ld_in + h * HD + d]);
    acc[d] = 0.f;
  }
  float m = -INFINITY, lsum = 0.f;
  const TB* bh = bias + (int64_t)h * N * N;
  for (int64_t k0 = 0; k0 < N; k0 += TK) {
    __syncthreads();
    for (int e = t; e < TK * HD; e += 256) {
      const int kk = e / HD, d = e - kk * HD;
      const bool in = k0 + kk < N;
      Ks[kk][d] = in ? to_f(k[(k0 + kk) * ld_in + h * HD + d]) : 0.f;
      Vs[kk][d] = in ? to_f(v[(k0 + kk) * ld_in + h * HD + d]) : 0.f;
    }
    for (int e = t; e < 16 * TK; e += 256) {
      const int qq = e / TK, kk = e - qq * TK;
      Bs[qq][kk] = (j0 + qq < N && k0 + kk < N) ? to_f(bh[(j0 + qq) * N + k0 + kk]) : 0.f;
    }
    if (t < TK) Mk[t] = k0 + t < N ? mask[k0 + t] : 0.f;
    __syncthreads();
#pragma unroll
    for (int u = 0; u < TK / 16; u++) {
      const int kk = 16 * u + kl;
      if (k0 + kk >= N) break;
      float sc = 0.f;
#pragma unroll
      for (int d = 0; d < HD; d++) sc += qv[d] * Ks[kk][d];
      sc = sc * scale + Bs[qi][kk];
      sc += (1.0f - Mk[kk]) * (-inf);
      const float mn = fmaxf(m, sc);
      const float corr = __expf(m - mn);
      const float p = __expf(sc - mn);
      lsum = lsum * corr + p;
#pragma unroll
      for (int d = 0; d < HD; d++) acc[d] = acc[d] * corr + p * Vs[kk][d];
      m = mn;
    }
  }
  // merge the 16 key lanes of each query (lanes 16*qi' .. 16*qi'+15 of the wave)
  float mt = m;
#pragma unroll
  for (int o = 8; o > 0; o >>= 1) mt = fmaxf(mt, __shfl_xor(mt, o, 64));
  const float f = (m == -INFINITY) ? 0.f : __expf(m - mt);
  lsum *= f;
#pragma unroll
  for (int o = 8; o > 0; o >>= 1) lsum += __shfl_xor(lsum, o, 64);
#pragma unroll
  for (int d = 0; d < HD; d++) {
    float a = acc[d] * f;
#pragma unroll
    for (int o = 8; o > 0; o >>= 1) a += __shfl_xor(a, o, 64);
    acc[d] = a;
  }
  if (!valid || kl != 0) return;
  const float inv = 1.0f / lsum;
#pragma unroll
  for (int d = 0; d < HD; d++)
    out[j * ld_out + h * HD + d] = from_f<T>(acc[d] * inv * sigmoidf_(to_f(g[j * ld_in + h * HD + d])));
}

template <typename T, typename TB>
static hipError_t seq_attn_t(const void* q, const void* k, const void* v, const void* g, int64_t ld_in,
                             const void* bias, const float* mask, float inf, void* out, int64_t ld_out, int64_t N,
                             int H, int hd, hipStream_t st) {
  const dim3 grid((unsigned)((N + 15) / 16), (unsigned)H);
  const float scale = 1.0f / sqrtf((float)hd);
#define BZ_SEQ(HDV)                                                                                              \
  seq_attn_kernel<T, TB, HDV><<<grid, 256, 0, st>>>(static_cast<const T*>(q), static_cast<const T*>(k),        \
                                                    static_cast<const T*>(v), static_cast<const T*>(g), ld_in,  \
                                                    static_cast<const TB*>(bias), mask, inf,                    \
                                                    static_cast<T*>(out), ld_out, N, scale)
  switch (hd) {
    case 16: BZ_SEQ(16); break;
    case 24: BZ_SEQ(24); break;
    case 32: BZ_SEQ(32); break;
    case 48: BZ_SEQ(48); break;
    case 64: BZ_SEQ(64); break;
    default: return hipErrorInvalidValue;
  }
#undef BZ_SEQ
  return hipGetLastError();
}

template <typename T>
static hipError_t core_valu_t(const void* qkg, const void* vt, const void* tb, const float* mask, int64_t mask_si,
                              int64_t mask_sk, float inf, void* out, int64_t N, int64_t ldk, int H, int C,
                              hipStream_t st) {
  const dim3 grid((unsigned)((N + 63) / 64), (unsigned)H, (unsigned)N);
  const T* q = static_cast<const T*>(qkg);
  const T* v = static_cast<const T*>(vt);
  const T* b = static_cast<const T*>(tb);
  T* o = static_cast<T*>(out);
  switch (C) {
    case 16: triattn_core_valu<T, 16><<<grid, 64, 0, st>>>(q, v, b, mask, mask_si, mask_sk, inf, o, N, ldk, H); break;
    case 32: triattn_core_valu<T, 32><<<grid, 64, 0, st>>>(q, v, b, mask, mask_si, mask_sk, inf, o, N, ldk, H); break;
    case 64: triattn_core_valu<T, 64><<<grid, 64, 0, st>>>(q, v, b, mask, mask_si, mask_sk, inf, o, N, ldk, H); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_triattn_core_simple(const void* qkg, const void* vt, const void* tb, const float* mask,
                                      int64_t mask_si, int64_t mask_sk, float inf, void* out, int dt, int64_t N,
                                      int64_t ldk, int H, int C, hipStream_t st) {
  return dt == DT_F16 ? core_valu_t<half_t>(qkg, vt, tb, mask, mask_si, mask_sk, inf, out, N, ldk, H, C, st)
                      : core_valu_t<float>(qkg, vt, tb, mask, mask_si, mask_sk, inf, out, N, ldk, H, C, st);
}

// Head widths 16, 24, 32, 48 and 64 (with the alignment their vector loads need) run on the matrix cores, all S
// samples in one launch: fp16 with an fp16 bias on bzpf_seqattn_mfma.hip, fp32 (with an fp32 or fp16 bias) on
// bzpf_seqattn_f32.hip. fp16 with an fp32 bias and other widths run on the VALU kernel above, one launch per
// sample.
hipError_t launch_seq_attention(const void* q, const void* k, const void* v, const void* g, int64_t ld_in,
                                int64_t s_in, const void* bias, int64_t s_bias, int mult, const float* mask,
                                int64_t s_mask, float inf, void* out, int64_t ld_out, int64_t s_out, int dt,
                                int bias_dt, int S, int64_t N, int H, int hd, hipStream_t st) {
  const auto al = [](const void* p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0; };
  if (S < 1 || mult < 1) return hipErrorInvalidValue;
  if (dt == DT_F16 && bias_dt == DT_F16 && (hd == 16 || hd == 24 || hd == 32 || hd == 48 || hd == 64) && N % 4 == 0 && ld_in % 8 == 0 &&
      ld_out % 4 == 0 && s_in % 8 == 0 && s_bias % 4 == 0 && s_out % 4 == 0 && al(q, 16) && al(k, 16) &&
      al(v, 16) && al(g, 16) && al(bias, 8) && al(out, 8) && S <= 65535 && seqattn_shape_ok(N, ld_in))
    return launch_seq_attention_f16_mfma(q, k, v, g, ld_in, s_in, bias, s_bias, mult, mask, s_mask, inf, out, ld_out,
                                         s_out, S, N, H, hd, st);
  if (dt == DT_F32 && (hd == 16 || hd == 24 || hd == 32 || hd == 48 || hd == 64) && ld_in % 4 == 0 &&
      s_in % 4 == 0 && al(q, 16) && al(k, 16) && al(v, 16) && al(g, 16) && N <= 46340 && S <= 65535)
    return launch_seq_attention_f32_mfma(q, k, v, g, ld_in, s_in, bias, s_bias, mult, mask, s_mask, inf, out, ld_out,
                                         s_out, bias_dt, S, N, H, hd, st);
  const int64_t es = dt == DT_F16 ? 2 : 4, esb = bias_dt == DT_F16 ? 2 : 4;
  const auto launch = dt == DT_F16 ? (bias_dt == DT_F16 ? seq_attn_t<half_t, half_t> : seq_attn_t<half_t, float>)
                                   : (bias_dt == DT_F16 ? seq_attn_t<float, half_t> : seq_attn_t<float, float>);
  for (int smp = 0; smp < S; smp++) {
    const int64_t oi = smp * s_in * es, ob = (int64_t)(smp / mult) * s_bias * esb, oo = smp * s_out * es;
    const auto at = [](const void* p, int64_t off) { return static_cast<const void*>(static_cast<const char*>(p) + off); };
    const hipError_t e = launch(at(q, oi), at(k, oi), at(v, oi), at(g, oi), ld_in, at(bias, ob), mask + smp * s_mask,
                                inf, static_cast<char*>(out) + oo, ld_out, N, H, hd, st);
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

// Core dispatch (impl mirrors the reference's scalar / mma choice, boltz_mlx/kernels.py:902-945): 0 = MFMA for
// fp16 with C = 32, else the VALU kernel; 1 = the VALU kernel; 2 = MFMA (fp16, C = 32 only).
hipError_t launch_triattn_core(const void* qkg, const void* vt, const void* tb, const float* mask, int64_t mask_si,
                               int64_t mask_sk, float inf, void* out, int dt, int64_t N, int64_t ldk, int H, int C,
                               int impl, hipStream_t st) {
  const bool mfma_ok = dt == DT_F16 && C == 32;
  if (impl == 2 && !mfma_ok) return hipErrorInvalidValue;
  if ((impl == 0 && mfma_ok) || impl == 2)
    return launch_triattn_core_f16_mfma(qkg, vt, tb, mask, mask_si, mask_sk, inf, out, N, ldk, H, C, st);
  return launch_triattn_core_simple(qkg, vt, tb, mask, mask_si, mask_sk, inf, out, dt, N, ldk, H, C, st);
}

}  // namespace bzpf
