// Triangle attention (starting and ending node) as three kernels:
//   proj  : q|k|v|g planes [4H][N*N][C] and the triangle bias tb [H][N*N] from the LayerNorm output, reading the
//           positions transposed for the ending node (so the core never sees the orientation);
//   core  : per row i and head h, out[i, j, h*C:(h+1)*C] = sigmoid(g) * softmax_k(q.k/sqrt(C) + inf*(mask-1) + tb)
//           v, flash-style with online softmax (a reference VALU kernel here; the fp16 MFMA kernel is in
//           bzpf_triattn_mfma.hip);
//   linear_resid_ln : z[src(p)] (+)= out[p] W_o^T, then the next LayerNorm of the updated row.
// Reference behaviour: boltz_mlx/layers/triangular_attention/attention.py:27-93 (fp32), 95-190 (f16),
// primitives.py:40-75 (q scaled before q.k; logits + mask_bias + tri_bias), kernels.py:538-600 (summation order
// (qk + mask_bias) + tri_bias), kernels_nax3.py:176-198 (linear_o + residual + next LN, transposed read of z).
#include "bzpf_common.h"
#include "bzpf_kernels.h"

namespace bzpf {

// ---------------------------------------------------------------- projection
// grid: (ceil(N^2 / 64) position tiles, ceil(M / 64) column chunks), M = 4*H*C + H; block 256.
// Outputs (position p = i*N + j of the attention frame; trans reads xn at (j, i)):
//   qkg [3H][N*N][C]   q (times q_scale), k, g planes, C contiguous channels per position;
//   vt  [H][N][C][ldk] v transposed per row i (keys contiguous), columns j >= N left unwritten;
//   tb  [H][N][ldk]    tri bias (times b_scale) for query j, key k of row-independent head h.
template <typename T>
__global__ __launch_bounds__(256) void triattn_proj_kernel(const T* __restrict__ xn, const T* __restrict__ w,
                                                           int trans, float q_scale, float b_scale,
                                                           T* __restrict__ qkg, T* __restrict__ vt,
                                                           T* __restrict__ tb, int64_t N, int64_t ldk, int H, int C) {
  constexpr int D = 128, PAD = Pad<T>::v, LDX = D + PAD, LDO = 64 + PAD;
  __shared__ LDS_ALIGN T Xs[64 * LDX];
  __shared__ LDS_ALIGN T Ws[64 * LDX];
  __shared__ LDS_ALIGN T Os[64 * LDO];
  const int64_t NN = N * N;
  const int64_t p0 = (int64_t)blockIdx.x * 64;
  const int HC = H * C, M = 4 * HC + H;
  const int c0 = blockIdx.y * 64;
  const int wave = threadIdx.x >> 6, l = threadIdx.x & 63;
  const int rows = (int)((NN - p0) < 64 ? (NN - p0) : 64);

  load_rows<T>(Xs, LDX, 64, D, [&](int r) -> const T* {
    int64_t p = p0 + (r < rows ? r : rows - 1);
    if (trans) { const int64_t i = p / N, j = p - i * N; p = j * N + i; }
    return xn + p * D;
  });
  load_rows<T>(Ws, LDX, 64, D, [&](int r) -> const T* { return (c0 + r < M) ? w + (int64_t)(c0 + r) * D : nullptr; });
  __syncthreads();
  f4 acc[1][4];
  zero_acc(acc);
  wave_mma<T, 1, 4>(acc, Xs + 16 * wave * LDX, LDX, Ws, LDX, D);
  const int plane4 = c0 / HC;  // 0 q, 1 k, 2 v, 3 g, 4 tri bias (chunks never straddle planes: HC % 64 == 0)
  const float sc = plane4 == 0 ? q_scale : (plane4 == 4 ? b_scale : 1.0f);
#pragma unroll
  for (int nb = 0; nb < 4; nb++)
#pragma unroll
    for (int e = 0; e < 4; e++)
      Os[(16 * wave + (l >> 4) * 4 + e) * LDO + 16 * nb + (l & 15)] = from_f<T>(acc[0][nb][e] * sc);
  __syncthreads();
  if (plane4 == 0 || plane4 == 1 || plane4 == 3) {
    // 64 / C plane-heads of C contiguous channels per position
    constexpr int VE = Vec16<T>::n;
    const int vpr = C / VE;
    const int nph = 64 / C;
    const int pl0 = (plane4 == 3 ? 2 : plane4) * H + (c0 - plane4 * HC) / C;
    for (int e = threadIdx.x; e < nph * 64 * vpr; e += 256) {
      const int ph = e / (64 * vpr);
      const int rem = e - ph * 64 * vpr;
      const int r = rem / vpr, d = (rem - r * vpr) * VE;
      if (r >= rows) continue;
      T* dst = qkg + ((int64_t)(pl0 + ph) * NN + p0 + r) * C + d;
      *reinterpret_cast<U128*>(dst) = *reinterpret_cast<const U128*>(Os + r * LDO + ph * C + d);
    }
  } else if (plane4 == 2) {
    // v transposed: consecutive lanes take consecutive positions (coalesced along keys)
    const int r = threadIdx.x & 63, cg = threadIdx.x >> 6;
    if (r < rows) {
      const int64_t p = p0 + r, i = p / N, j = p - i * N;
#pragma unroll 4
      for (int u = 0; u < 16; u++) {
        const int col = c0 - 2 * HC + cg * 16 + u;  // channel within the v plane group
        const int hh = col / C, d = col - hh * C;
        vt[(((int64_t)hh * N + i) * C + d) * ldk + j] = Os[r * LDO + cg * 16 + u];
      }
    }
  } else {
    for (int e = threadIdx.x; e < H * 64; e += 256) {
      const int hh = e / 64, r = e - hh * 64;
      if (r < rows && c0 + hh < M) {
        const int64_t p = p0 + r, i = p / N, j = p - i * N;
        T* row = tb + ((int64_t)hh * N + i) * ldk;
        row[j] = Os[r * LDO + (4 * HC + hh - c0)];
        if (j == N - 1)  // finite padding: the MFMA core adds it before masking the keys past N with -inf
          for (int64_t k = N; k < ldk; k++) row[k] = from_f<T>(0.0f);
      }
    }
  }
}

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

// ---------------------------------------------------------------- linear_o + residual + next LN
// grid: ceil(N^2 / 64) position tiles; block 256 (wave w: rows 16w..16w+15, all 128 columns).
template <typename T>
__global__ __launch_bounds__(256) void linear_resid_ln_kernel(const T* __restrict__ x, const T* __restrict__ w,
                                                              int trans, float* __restrict__ z, int accumulate,
                                                              const float* __restrict__ lnw,
                                                              const float* __restrict__ lnb, float eps,
                                                              T* __restrict__ xn_next, int64_t N) {
  constexpr int D = 128, PAD = Pad<T>::v, LDX = D + PAD, LDY = D + 4;
  constexpr int X_BYTES = 64 * LDX * (int)sizeof(T), Y_BYTES = 64 * LDY * 4;
  __shared__ LDS_ALIGN char smem[X_BYTES > Y_BYTES ? X_BYTES : Y_BYTES];
  __shared__ LDS_ALIGN T Ws[64 * LDX];
  T* Xs = reinterpret_cast<T*>(smem);
  float* Ys = reinterpret_cast<float*>(smem);
  const int64_t NN = N * N;
  const int64_t p0 = (int64_t)blockIdx.x * 64;
  const int rows = (int)((NN - p0) < 64 ? (NN - p0) : 64);
  const int wave = threadIdx.x >> 6, l = threadIdx.x & 63;
  load_rows<T>(Xs, LDX, 64, D, [&](int r) { return x + (p0 + (r < rows ? r : rows - 1)) * D; });
  f4 acc[1][8];
  zero_acc(acc);
  for (int cc = 0; cc < 2; cc++) {
    __syncthreads();
    load_rows<T>(Ws, LDX, 64, D, [&](int r) { return w + (int64_t)(64 * cc + r) * D; });
    __syncthreads();
    f4 t4[1][4];
    zero_acc(t4);
    wave_mma<T, 1, 4>(t4, Xs + 16 * wave * LDX, LDX, Ws, LDX, D);
#pragma unroll
    for (int nb = 0; nb < 4; nb++) acc[0][4 * cc + nb] = t4[0][nb];
  }
  __syncthreads();
#pragma unroll
  for (int nb = 0; nb < 8; nb++)
#pragma unroll
    for (int e = 0; e < 4; e++) Ys[(16 * wave + (l >> 4) * 4 + e) * LDY + 16 * nb + (l & 15)] = acc[0][nb][e];
  __syncthreads();
  resid_ln_epilogue<T>(Ys, LDY, rows, [&](int r) -> int64_t {
    int64_t p = p0 + r;
    if (trans) { const int64_t i = p / N, j = p - i * N; p = j * N + i; }
    return p;
  }, z, accumulate, lnw, lnb, eps, xn_next);
}

template <typename T>
static hipError_t proj_t(const void* xn, const void* w, int trans, float q_scale, float b_scale, void* qkg, void* vt,
                         void* tb, int64_t N, int64_t ldk, int H, int C, hipStream_t st) {
  const int M = 4 * H * C + H;
  const dim3 grid((unsigned)((N * N + 63) / 64), (unsigned)((M + 63) / 64));
  triattn_proj_kernel<T><<<grid, 256, 0, st>>>(static_cast<const T*>(xn), static_cast<const T*>(w), trans, q_scale,
                                               b_scale, static_cast<T*>(qkg), static_cast<T*>(vt), static_cast<T*>(tb),
                                               N, ldk, H, C);
  return hipGetLastError();
}

hipError_t launch_triattn_proj(const void* xn, const void* w, int trans, float q_scale, float b_scale, void* qkg,
                               void* vt, void* tb, int dt, int64_t N, int64_t ldk, int H, int C, hipStream_t st) {
  return dt == DT_F16 ? proj_t<half_t>(xn, w, trans, q_scale, b_scale, qkg, vt, tb, N, ldk, H, C, st)
                      : proj_t<float>(xn, w, trans, q_scale, b_scale, qkg, vt, tb, N, ldk, H, C, st);
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

template <typename T>
static hipError_t lrl_t(const void* x, const void* w, int trans, float* z, int accumulate, const float* lnw,
                        const float* lnb, float eps, void* xn_next, int64_t N, hipStream_t st) {
  const dim3 grid((unsigned)((N * N + 63) / 64));
  linear_resid_ln_kernel<T><<<grid, 256, 0, st>>>(static_cast<const T*>(x), static_cast<const T*>(w), trans, z,
                                                  accumulate, lnw, lnb, eps, static_cast<T*>(xn_next), N);
  return hipGetLastError();
}

hipError_t launch_linear_resid_ln(const void* x, const void* w, int trans, float* z, int accumulate,
                                  const float* lnw, const float* lnb, float eps, void* xn_next, int dt, int64_t N,
                                  hipStream_t st) {
  return dt == DT_F16 ? lrl_t<half_t>(x, w, trans, z, accumulate, lnw, lnb, eps, xn_next, N, st)
                      : lrl_t<float>(x, w, trans, z, accumulate, lnw, lnb, eps, xn_next, N, st);
}

}  // namespace bzpf

namespace bzpf {

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
