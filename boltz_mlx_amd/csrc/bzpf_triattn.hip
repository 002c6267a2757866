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
  const T* bb = tb + h * N * ldk;
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
      Bs[qq][kk] = (j0 + qq < N && k0 + kk < N) ? to_f(bb[(j0 + qq) * ldk + k0 + kk]) : 0.f;
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
// One thread per query j; a 64-thread workgroup owns (head h, 64 queries). Keys are staged TK at a time in LDS
// (K, V and the [64 x TK] bias tile, all loaded coalesced). order 0: s = (q*scale).k, s += inf*(m-1), s += bias;
// order 1 (AttentionPairBias, attentionv2.py:76-81): s = (q.k)*scale + bias, s += (1-m)*(-inf). Element (row i, position j, head h, channel d) of q/k/v/g is at
// base + i*s_row + j*s_pos + h*s_head + d; the output uses o_row/o_pos/o_head.
struct AttnArgs {
  const void *q, *k, *v, *g, *bias;
  const float* mask;
  void* out;
  int64_t s_row, s_pos, s_head;
  int64_t o_row, o_pos, o_head;
  int64_t b_head;        // bias head stride (bias[h*b_head + j*J + k])
  int64_t m_row, m_key;  // mask strides
  float inf, scale;
  int64_t J;
  int order;
};

template <typename T, int HD>
__global__ __launch_bounds__(64) void attn_simple_kernel(AttnArgs a) {
  constexpr int TK = 32;
  __shared__ float Ks[TK][HD + 1];
  __shared__ float Vs[TK][HD + 1];
  __shared__ float Bs[64][TK + 1];
  __shared__ float Mk[TK];
  const int64_t J = a.J;
  const int t = threadIdx.x;
  const int64_t j = (int64_t)blockIdx.x * 64 + t;
  const int64_t h = blockIdx.y, i = blockIdx.z;
  const bool valid = j < J;
  const T* qb = static_cast<const T*>(a.q) + i * a.s_row + h * a.s_head;
  const T* kb = static_cast<const T*>(a.k) + i * a.s_row + h * a.s_head;
  const T* vb = static_cast<const T*>(a.v) + i * a.s_row + h * a.s_head;
  const T* bb = static_cast<const T*>(a.bias) + h * a.b_head;
  float q[HD], acc[HD];
#pragma unroll
  for (int d = 0; d < HD; d++) {
    const float qv = valid ? to_f(qb[j * a.s_pos + d]) : 0.f;
    q[d] = a.order == 0 ? qv * a.scale : qv;
    acc[d] = 0.f;
  }
  float m = -INFINITY, lsum = 0.f;
  const int64_t j0 = (int64_t)blockIdx.x * 64;
  for (int64_t k0 = 0; k0 < J; k0 += TK) {
    __syncthreads();
    for (int e = t; e < TK * HD; e += 64) {
      const int kk = e / HD, d = e - kk * HD;
      const int64_t key = k0 + kk;
      Ks[kk][d] = key < J ? to_f(kb[key * a.s_pos + d]) : 0.f;
      Vs[kk][d] = key < J ? to_f(vb[key * a.s_pos + d]) : 0.f;
    }
    for (int e = t; e < 64 * TK; e += 64) {
      const int qq = e / TK, kk = e - qq * TK;
      const int64_t jq = j0 + qq, key = k0 + kk;
      Bs[qq][kk] = (jq < J && key < J) ? to_f(bb[jq * J + key]) : 0.f;
    }
    if (t < TK) {
      const int64_t key = k0 + t;
      Mk[t] = key < J ? a.mask[i * a.m_row + key * a.m_key] : 0.f;
    }
    __syncthreads();
    const int kend = (int)((J - k0) < TK ? (J - k0) : TK);
    for (int kk = 0; kk < kend; kk++) {
      float s = 0.f;
#pragma unroll
      for (int d = 0; d < HD; d++) s += q[d] * Ks[kk][d];
      if (a.order == 0) {
        s += a.inf * (Mk[kk] - 1.0f);
        s += Bs[t][kk];
      } else {
        s = s * a.scale + Bs[t][kk];
        s += (1.0f - Mk[kk]) * (-a.inf);
      }
      const float mn = fmaxf(m, s);
      const float corr = __expf(m - mn);
      const float p = __expf(s - mn);
      lsum = lsum * corr + p;
#pragma unroll
      for (int d = 0; d < HD; d++) acc[d] = acc[d] * corr + p * Vs[kk][d];
      m = mn;
    }
  }
  if (!valid) return;
  const float inv = 1.0f / lsum;
  const T* gb = static_cast<const T*>(a.g) + i * a.s_row + h * a.s_head + j * a.s_pos;
  T* ob = static_cast<T*>(a.out) + i * a.o_row + j * a.o_pos + h * a.o_head;
#pragma unroll
  for (int d = 0; d < HD; d++) ob[d] = from_f<T>(acc[d] * inv * sigmoidf_(to_f(gb[d])));
}

template <typename T>
static hipError_t attn_simple_launch(const AttnArgs& a, int64_t rows, int H, int hd, hipStream_t st) {
  const dim3 grid((unsigned)((a.J + 63) / 64), (unsigned)H, (unsigned)rows);
  switch (hd) {
    case 16: attn_simple_kernel<T, 16><<<grid, 64, 0, st>>>(a); break;
    case 24: attn_simple_kernel<T, 24><<<grid, 64, 0, st>>>(a); break;
    case 32: attn_simple_kernel<T, 32><<<grid, 64, 0, st>>>(a); break;
    case 48: attn_simple_kernel<T, 48><<<grid, 64, 0, st>>>(a); break;
    case 64: attn_simple_kernel<T, 64><<<grid, 64, 0, st>>>(a); break;
    default: return hipErrorInvalidValue;
  }
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

hipError_t launch_seq_attention(const void* q, const void* k, const void* v, const void* g, int64_t ld_in,
                                const void* bias, const float* mask, float inf, void* out, int64_t ld_out, int dt,
                                int64_t N, int H, int hd, hipStream_t st) {
  AttnArgs a;
  a.q = q; a.k = k; a.v = v; a.g = g;
  a.bias = bias;
  a.mask = mask;
  a.out = out;
  a.s_row = 0; a.s_pos = ld_in; a.s_head = hd;
  a.o_row = 0; a.o_pos = ld_out; a.o_head = hd;
  a.b_head = N * N;
  a.m_row = 0; a.m_key = 1;
  a.inf = inf;
  a.scale = 1.0f / sqrtf((float)hd);
  a.J = N;
  a.order = 1;
  return dt == DT_F16 ? attn_simple_launch<half_t>(a, 1, H, hd, st) : attn_simple_launch<float>(a, 1, H, hd, st);
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
