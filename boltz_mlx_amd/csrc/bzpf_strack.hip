// Sequence-track (s) kernels of the PairformerLayer and the pair bias it reads from z:
//   linear    : Y = X W^T (+ bias) with an fp32 residual-accumulate option (tiled MFMA, any K % 8 == 0);
//   swiglu    : a = silu(h[:, :H]) * h[:, H:];  swiglu3: a = silu(h[:, :H]) * h[:, H:2H] * h[:, 2H:];
//   adaln     : sigmoid(scale) * LN(a) + shift (the diffusion transformer's conditioned LayerNorm);
//   pair_bias : bias[h][p] = LN(z[p]) . W[h] over all N*N pair positions (proj_z).
// Reference behaviour: boltz_mlx/layers/attentionv2.py:43-86 (AttentionPairBias), transition.py:27-54 and
// 148-154 (Transition on s), pairformer.py:90-93 (s-track residuals).
#include "bzpf_common.h"
#include "bzpf_kernels.h"

namespace bzpf {

// ---------------------------------------------------------------- generic linear
// grid (ceil(R/64), ceil(M/64)); block 256; wave w: rows 16w..16w+15 of the tile, 64 columns. epi 0: y = acc + b
// (stored as TY); epi 1: y (fp32) += acc + b.
template <typename T, typename TY>
__global__ __launch_bounds__(256) void linear_kernel(const T* __restrict__ x, const T* __restrict__ w,
                                                     const float* __restrict__ bias, TY* __restrict__ y, int64_t R,
                                                     int K, int M, int epi, const float* __restrict__ gate,
                                                     int64_t ld_gate, int64_t gate_rows) {
  constexpr int BK = 32, PAD = Pad<T>::v, LDK = BK + PAD, VE = Vec16<T>::n;
  __shared__ LDS_ALIGN T Xs[64 * LDK];
  __shared__ LDS_ALIGN T Ws[64 * LDK];
  const int64_t r0 = (int64_t)blockIdx.x * 64;
  const int c0 = blockIdx.y * 64;
  const int wave = threadIdx.x >> 6, l = threadIdx.x & 63;
  f4 acc[1][4];
  zero_acc(acc);
  for (int k0 = 0; k0 < K; k0 += BK) {
    __syncthreads();
    for (int e = threadIdx.x; e < 2 * 64 * (BK / VE); e += 256) {
      const int which = e / (64 * (BK / VE));
      const int rem = e - which * 64 * (BK / VE);
      const int r = rem / (BK / VE), kk = (rem - r * (BK / VE)) * VE;
      U128 v = U128{{0u, 0u, 0u, 0u}};
      if (k0 + kk < K) {
        if (which == 0) {
          int64_t rr = r0 + r;
          if (rr >= R) rr = R - 1;
          v = *reinterpret_cast<const U128*>(x + rr * K + k0 + kk);
        } else if (c0 + r < M) {
          v = *reinterpret_cast<const U128*>(w + (int64_t)(c0 + r) * K + k0 + kk);
        }
      }
      *reinterpret_cast<U128*>((which == 0 ? Xs : Ws) + r * LDK + kk) = v;
    }
    __syncthreads();
    wave_mma<T, 1, 4>(acc, Xs + 16 * wave * LDK, LDK, Ws, LDK, BK);
  }
#pragma unroll
  for (int nb = 0; nb < 4; nb++)
#pragma unroll
    for (int e = 0; e < 4; e++) {
      const int64_t r = r0 + 16 * wave + (l >> 4) * 4 + e;
      const int c = c0 + 16 * nb + (l & 15);
      if (r < R && c < M) {
        float v = acc[0][nb][e] + (bias ? bias[c] : 0.f);
        if (epi == 2) v *= sigmoidf_(gate[(r % gate_rows) * ld_gate + c]);
        if (epi >= 1) v += to_f(y[r * M + c]);
        y[r * M + c] = from_f<TY>(v);
      }
    }
}

template <typename T, typename TY>
static hipError_t linear_t(const void* x, const void* w, const float* bias, void* y, int64_t R, int K, int M, int epi,
                           const float* gate, int64_t ld_gate, int64_t gate_rows, hipStream_t st) {
  const dim3 grid((unsigned)((R + 63) / 64), (unsigned)((M + 63) / 64));
  linear_kernel<T, TY><<<grid, 256, 0, st>>>(static_cast<const T*>(x), static_cast<const T*>(w), bias,
                                             static_cast<TY*>(y), R, K, M, epi, gate, ld_gate, gate_rows);
  return hipGetLastError();
}

hipError_t launch_linear(const void* x, const void* w, const float* bias, void* y, int dt, int y_dt, int64_t rows,
                         int K, int M, int epi, hipStream_t st) {
  if (K % 8 || epi < 0 || epi > 1) return hipErrorInvalidValue;
  if (epi == 1 && y_dt != DT_F32) return hipErrorInvalidValue;
  if (gemm_nt_ok(dt, x, w, bias, y, rows, K, M, nullptr, 0))
    return launch_gemm_nt(x, w, bias, y, dt, y_dt, rows, K, M, epi, nullptr, 0, 1, st);
  if (dt == DT_F16) {
    return y_dt == DT_F16 ? linear_t<half_t, half_t>(x, w, bias, y, rows, K, M, epi, nullptr, 0, 1, st)
                          : linear_t<half_t, float>(x, w, bias, y, rows, K, M, epi, nullptr, 0, 1, st);
  }
  return y_dt == DT_F16 ? linear_t<float, half_t>(x, w, bias, y, rows, K, M, epi, nullptr, 0, 1, st)
                        : linear_t<float, float>(x, w, bias, y, rows, K, M, epi, nullptr, 0, 1, st);
}

hipError_t launch_linear_gated(const void* x, const void* w, const float* bias, const float* gate, int64_t ld_gate,
                               int64_t gate_rows, float* y, int dt, int64_t rows, int K, int M, hipStream_t st) {
  if (K % 8 || gate_rows < 1) return hipErrorInvalidValue;
  if (gemm_nt_ok(dt, x, w, bias, y, rows, K, M, gate, ld_gate))
    return launch_gemm_nt(x, w, bias, y, dt, DT_F32, rows, K, M, 2, gate, ld_gate, gate_rows, st);
  return dt == DT_F16 ? linear_t<half_t, float>(x, w, bias, y, rows, K, M, 2, gate, ld_gate, gate_rows, st)
                      : linear_t<float, float>(x, w, bias, y, rows, K, M, 2, gate, ld_gate, gate_rows, st);
}

// ---------------------------------------------------------------- SwiGLU
template <typename T>
__global__ __launch_bounds__(256) void swiglu_kernel(const T* __restrict__ h, T* __restrict__ a, int64_t R, int H) {
  const int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (e >= R * H) return;
  const int64_t r = e / H, c = e - r * H;
  a[e] = from_f<T>(siluf_(to_f(h[r * 2 * H + c])) * to_f(h[r * 2 * H + H + c]));
}

hipError_t launch_swiglu(const void* h, void* a, int dt, int64_t R, int H, hipStream_t st) {
  const dim3 grid((unsigned)((R * H + 255) / 256));
  if (dt == DT_F16)
    swiglu_kernel<half_t><<<grid, 256, 0, st>>>(static_cast<const half_t*>(h), static_cast<half_t*>(a), R, H);
  else
    swiglu_kernel<float><<<grid, 256, 0, st>>>(static_cast<const float*>(h), static_cast<float*>(a), R, H);
  return hipGetLastError();
}

// a[r][c] = silu(h[r][c]) * h[r][H + c] * h[r][2H + c] (rows of h: 3H). The conditioned transition's gated product
// silu(gates) * x * a_to_b(a) with the GEMM rows ordered [gates; x; a_to_b] (transformersv2.py:44-66).
template <typename T>
__global__ __launch_bounds__(256) void swiglu3_kernel(const T* __restrict__ h, T* __restrict__ a, int64_t R, int H) {
  const int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (e >= R * H) return;
  const int64_t r = e / H, c = e - r * H;
  const T* hr = h + r * 3 * H;
  a[e] = from_f<T>(siluf_(to_f(hr[c])) * to_f(hr[H + c]) * to_f(hr[2 * H + c]));
}

hipError_t launch_swiglu3(const void* h, void* a, int dt, int64_t R, int H, hipStream_t st) {
  const dim3 grid((unsigned)((R * H + 255) / 256));
  if (dt == DT_F16)
    swiglu3_kernel<half_t><<<grid, 256, 0, st>>>(static_cast<const half_t*>(h), static_cast<half_t*>(a), R, H);
  else
    swiglu3_kernel<float><<<grid, 256, 0, st>>>(static_cast<const float*>(h), static_cast<float*>(a), R, H);
  return hipGetLastError();
}

// ---------------------------------------------------------------- AdaLN
// out[r][c] = sigmoid(scale[q][c]) * LN(a[r])[c] + shift[q][c], q = r % cond_rows (conditioning rows of pitch ldc),
// LN without affine (two-pass fp32 statistics). One wave per row, lane l holding columns l + 64 j.
// Reference: AdaLN (boltz_mlx/modules/transformersv2.py:27-41) with the s-side projections precomputed for all
// layers (transformersv2.py:400-420: sigmoid applied here, in the consumer).
template <typename TO, int NV>
__global__ __launch_bounds__(256) void adaln_kernel(const float* __restrict__ a, const float* __restrict__ scale,
                                                    const float* __restrict__ shift, int64_t ldc, int64_t cond_rows,
                                                    float eps, TO* __restrict__ out, int64_t R) {
  constexpr int D = 64 * NV;
  const int l = threadIdx.x & 63;
  const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (r >= R) return;  // whole wave
  const float* ar = a + r * D;
  // the conditioning row's scale and shift are loaded first: they do not depend on the statistics, so the row costs
  // one round trip to memory instead of two
  const int64_t q = r % cond_rows;
  const float* sc = scale + q * ldc;
  const float* sh = shift + q * ldc;
  float gs[NV], hs[NV];
#pragma unroll
  for (int j = 0; j < NV; j++) {
    gs[j] = sc[l + 64 * j];
    hs[j] = sh[l + 64 * j];
  }
  float v[NV];
  float s = 0.f;
#pragma unroll
  for (int j = 0; j < NV; j++) {
    v[j] = ar[l + 64 * j];
    s += v[j];
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) s += __shfl_xor(s, o, 64);
  const float mean = s * (1.0f / D);
  float ss = 0.f;
#pragma unroll
  for (int j = 0; j < NV; j++) {
    const float d = v[j] - mean;
    ss += d * d;
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) ss += __shfl_xor(ss, o, 64);
  const float rstd = 1.0f / sqrtf(ss * (1.0f / D) + eps);
  TO* orow = out + r * D;
#pragma unroll
  for (int j = 0; j < NV; j++) orow[l + 64 * j] = from_f<TO>(sigmoidf_(gs[j]) * ((v[j] - mean) * rstd) + hs[j]);
}

template <typename TO>
static hipError_t adaln_t(const float* a, const float* scale, const float* shift, int64_t ldc, int64_t cond_rows,
                          float eps, void* out, int64_t R, int D, hipStream_t st) {
  const dim3 grid((unsigned)((R + 3) / 4));
  TO* o = static_cast<TO*>(out);
  switch (D / 64) {
#define BZ_CASE(nv) \
  case nv: adaln_kernel<TO, nv><<<grid, 256, 0, st>>>(a, scale, shift, ldc, cond_rows, eps, o, R); break;
    BZ_CASE(1) BZ_CASE(2) BZ_CASE(3) BZ_CASE(4) BZ_CASE(6) BZ_CASE(8) BZ_CASE(12) BZ_CASE(16)
#undef BZ_CASE
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_adaln(const float* a, const float* scale, const float* shift, int64_t ldc, int64_t cond_rows,
                        float eps, void* out, int out_dt, int64_t R, int D, hipStream_t st) {
  if (D % 64 || cond_rows < 1) return hipErrorInvalidValue;
  return out_dt == DT_F16 ? adaln_t<half_t>(a, scale, shift, ldc, cond_rows, eps, out, R, D, st)
                          : adaln_t<float>(a, scale, shift, ldc, cond_rows, eps, out, R, D, st);
}

// ---------------------------------------------------------------- pair bias = Linear(LN(z)) as [H][rows]
// grid ceil(rows/64); block 256; H <= 16 heads, D = 128.
template <typename T>
__global__ __launch_bounds__(256) void pair_bias_kernel(const float* __restrict__ z, const float* __restrict__ lnw,
                                                        const float* __restrict__ lnb, float eps,
                                                        const T* __restrict__ w, T* __restrict__ out, int64_t rows_total,
                                                        int H) {
  constexpr int D = 128, PAD = Pad<T>::v, LDX = D + PAD, LDO = 64 + 4;
  __shared__ LDS_ALIGN T Xs[64 * LDX];
  __shared__ LDS_ALIGN T Ws[16 * LDX];
  __shared__ float Os[16 * LDO];
  const int64_t r0 = (int64_t)blockIdx.x * 64;
  const int rows = (int)((rows_total - r0) < 64 ? (rows_total - r0) : 64);
  const int wave = threadIdx.x >> 6, l = threadIdx.x & 63;
  {
    const int r = threadIdx.x >> 2, q = threadIdx.x & 3;
    const float* zr = z + (r0 + (r < rows ? r : rows - 1)) * D + q * 32;
    float v[32];
    float s = 0.f;
#pragma unroll
    for (int c = 0; c < 32; c += 4) {
      f4 t = *reinterpret_cast<const f4*>(zr + c);
      v[c] = t[0]; v[c + 1] = t[1]; v[c + 2] = t[2]; v[c + 3] = t[3];
      s += t[0] + t[1] + t[2] + t[3];
    }
    const float mean = group_sum<4>(s) * (1.0f / D);
    float ss = 0.f;
#pragma unroll
    for (int c = 0; c < 32; c++) { const float d = v[c] - mean; ss += d * d; }
    const float rstd = 1.0f / sqrtf(group_sum<4>(ss) * (1.0f / D) + eps);
#pragma unroll
    for (int c = 0; c < 32; c++)
      Xs[r * LDX + q * 32 + c] = from_f<T>((v[c] - mean) * rstd * lnw[q * 32 + c] + lnb[q * 32 + c]);
  }
  load_rows<T>(Ws, LDX, 16, D, [&](int r) -> const T* { return r < H ? w + (int64_t)r * D : nullptr; });
  __syncthreads();
  f4 acc[1][1];
  zero_acc(acc);
  wave_mma<T, 1, 1>(acc, Xs + 16 * wave * LDX, LDX, Ws, LDX, D);
#pragma unroll
  for (int e = 0; e < 4; e++) Os[(l & 15) * LDO + 16 * wave + (l >> 4) * 4 + e] = acc[0][0][e];
  __syncthreads();
  for (int e = threadIdx.x; e < H * 64; e += 256) {
    const int h = e >> 6, r = e & 63;
    if (r < rows) out[(int64_t)h * rows_total + r0 + r] = from_f<T>(Os[h * LDO + r]);
  }
}

hipError_t launch_pair_bias(const float* z, const float* lnw, const float* lnb, float eps, const void* w, void* out,
                            int dt, int64_t rows, int H, hipStream_t st) {
  if (H > 16) return hipErrorInvalidValue;
  const dim3 grid((unsigned)((rows + 63) / 64));
  if (dt == DT_F16)
    pair_bias_kernel<half_t><<<grid, 256, 0, st>>>(z, lnw, lnb, eps, static_cast<const half_t*>(w),
                                                   static_cast<half_t*>(out), rows, H);
  else
    pair_bias_kernel<float><<<grid, 256, 0, st>>>(z, lnw, lnb, eps, static_cast<const float*>(w),
                                                  static_cast<float*>(out), rows, H);
  return hipGetLastError();
}

}  // namespace bzpf
