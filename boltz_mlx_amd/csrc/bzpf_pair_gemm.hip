// The row-GEMM kernels of the pair track, all on the transposed row-tile scheme of bzpf_rowgemm.h (Y^T = W X^T with
// X rows in registers and W streamed through LDS in 64-channel chunks):
//   trimul_proj      : ab[c][i][k] = (xn W_p[c]) * sigmoid(xn W_g[c]) * mask * scale at (i, k) (incoming: (k, i))
//                      (boltz_mlx/layers/triangular_mult.py:67-88, 143-170; kernels_nax2.py:202-304);
//   trimul_tail      : z (+)= p_out(LN_out(o)) * sigmoid(g_out(xn)), then the next LayerNorm
//                      (triangular_mult.py:98-118; kernels_nax3.py:200-268, 1061-1206);
//   triattn_proj     : q|k|v|g planes, V^T rows and the triangle bias (attention.py:49-69, 100-104);
//   linear_resid_ln  : z (+)= x W_o^T at the (transposed) position, then the next LayerNorm (kernels_nax3.py:176-198);
//   transition       : z (+)= fc3(silu(fc1 xn) * fc2 xn), then the next LayerNorm (transition.py:27-54, 148-154;
//                      kernels_nax2.py:54-190, kernels_nax3.py:713-827).
// Tiles are 64 * RB rows (positions) per workgroup of 4 waves, RB = 2 row blocks per wave for fp16 and 1 for fp32.
#include "bzpf_common.h"
#include "bzpf_kernels.h"
#include "bzpf_rowgemm.h"

namespace bzpf {

namespace {

constexpr int D = 128;

template <typename T> constexpr int ldw_of() { return D + Pad<T>::v; }

// ---------------------------------------------------------------- triangle multiplication projection
// grid: N * tiles_per_row, tiles of TM positions (i, k0 .. k0+TM) of the padded row of length ld.
template <typename T>
__global__ __launch_bounds__(256) void trimul_proj_k(const T* __restrict__ xn, const T* __restrict__ w,
                                                     const float* __restrict__ mask, float scale, int incoming,
                                                     T* __restrict__ ab, int64_t N, int64_t ld) {
  constexpr int RB = RowBlocks<T>::v, TM = 64 * RB, STEPS = RG<T>::STEPS, LDW = ldw_of<T>();
  __shared__ LDS_ALIGN T Ws[64 * LDW];
  const int64_t tpr = (ld + TM - 1) / TM;
  const int64_t i = blockIdx.x / tpr;
  const int64_t k0 = (blockIdx.x - i * tpr) * TM;
  const int wave = threadIdx.x >> 6, l = threadIdx.x & 63, g = l >> 4;

  typename RG<T>::frag x[RB][STEPS];
  int64_t kpos[RB];
  float mk[RB];
#pragma unroll
  for (int rb = 0; rb < RB; rb++) {
    kpos[rb] = k0 + wave * 16 * RB + 16 * rb + (l & 15);
    const int64_t kc = kpos[rb] < N ? kpos[rb] : N - 1;
    const int64_t src = incoming ? (kc * N + i) : (i * N + kc);
    RG<T>::load_row(x[rb], xn + src * D, g);
    mk[rb] = kpos[rb] < N ? mask[src] * scale : 0.0f;  // padding columns k >= N are written as 0
  }
  for (int c0 = 0; c0 < 2 * D; c0 += 32) {
    __syncthreads();
    lds_rows<T>(Ws, LDW, 64, D, [&](int r) { return w + (int64_t)(r < 32 ? c0 + r : 2 * D + c0 + r - 32) * D; });
    __syncthreads();
    f4 acc[RB][4];
    zero_acc(acc);
    mma_rows<T, RB, 4>(acc, x, Ws, LDW);
#pragma unroll
    for (int rb = 0; rb < RB; rb++) {
      if (kpos[rb] >= ld) continue;
#pragma unroll
      for (int cb = 0; cb < 2; cb++)
#pragma unroll
        for (int e = 0; e < 4; e++) {
          const int ch = c0 + 16 * cb + 4 * g + e;
          const float v = acc[rb][cb][e] * sigmoidf_(acc[rb][cb + 2][e]) * mk[rb];
          ab[((int64_t)ch * N + i) * ld + kpos[rb]] = from_f<T>(v);
        }
    }
  }
}

// ---------------------------------------------------------------- triangle multiplication tail
// grid: N * tiles_per_row over the padded rows (positions (i, j0 .. j0+TM)).
template <typename T>
__global__ __launch_bounds__(256) void trimul_tail_k(const T* __restrict__ o, const float* __restrict__ now,
                                                     const float* __restrict__ nob, float eps_out,
                                                     const T* __restrict__ w_po, const T* __restrict__ xn,
                                                     const T* __restrict__ w_go, float* __restrict__ z, int accumulate,
                                                     const float* __restrict__ lnw, const float* __restrict__ lnb,
                                                     float eps_next, T* __restrict__ xn_next, int64_t N, int64_t ld) {
  constexpr int RB = RowBlocks<T>::v, TM = 64 * RB, STEPS = RG<T>::STEPS, LDW = ldw_of<T>();
  __shared__ LDS_ALIGN T Ts[TM * LDW];  // o tile transposed to [position][channel], then LN_out of it
  __shared__ LDS_ALIGN T Ws[64 * LDW];
  const int64_t tpr = (ld + TM - 1) / TM;
  const int64_t i = blockIdx.x / tpr;
  const int64_t j0 = (blockIdx.x - i * tpr) * TM;
  const int wave = threadIdx.x >> 6, l = threadIdx.x & 63, g = l >> 4;

  // o tile: each channel row holds contiguous positions (columns past ld are not read)
  {
    constexpr int VE = Vec16<T>::n;
    for (int e = threadIdx.x; e < D * (TM / VE); e += 256) {
      const int c = e / (TM / VE), r = (e - c * (TM / VE)) * VE;
      if (j0 + r >= ld) continue;
      U128 v = *reinterpret_cast<const U128*>(o + ((int64_t)c * N + i) * ld + j0 + r);
      const T* vv = reinterpret_cast<const T*>(&v);
#pragma unroll
      for (int u = 0; u < VE; u++) Ts[(r + u) * LDW + c] = vv[u];
    }
  }
  __syncthreads();
  // LN_out over the 128 channels of each position (4 threads per row, two-pass fp32 statistics)
  for (int r = threadIdx.x >> 2; r < TM; r += 64) {
    const int q = threadIdx.x & 3;
    T* tr = Ts + r * LDW + q * 32;
    float v[32];
    float s = 0.f;
#pragma unroll
    for (int c = 0; c < 32; c++) { v[c] = to_f(tr[c]); s += v[c]; }
    const float mean = group_sum<4>(s) * (1.0f / D);
    float ss = 0.f;
#pragma unroll
    for (int c = 0; c < 32; c++) { const float d = v[c] - mean; ss += d * d; }
    const float rstd = 1.0f / sqrtf(group_sum<4>(ss) * (1.0f / D) + eps_out);
#pragma unroll
    for (int c = 0; c < 32; c++) tr[c] = from_f<T>((v[c] - mean) * rstd * now[q * 32 + c] + nob[q * 32 + c]);
  }
  int64_t jpos[RB];
  typename RG<T>::frag x[RB][STEPS];
#pragma unroll
  for (int rb = 0; rb < RB; rb++) {
    jpos[rb] = j0 + wave * 16 * RB + 16 * rb + (l & 15);
    const int64_t jc = jpos[rb] < N ? jpos[rb] : N - 1;
    RG<T>::load_row(x[rb], xn + (i * N + jc) * D, g);
  }
  // gates sigmoid(xn W_go^T), two 64-channel chunks
  f4 gate[RB][8];
#pragma unroll
  for (int cc = 0; cc < 2; cc++) {
    __syncthreads();
    lds_rows<T>(Ws, LDW, 64, D, [&](int r) { return w_go + (int64_t)(64 * cc + r) * D; });
    __syncthreads();
    f4 acc[RB][4];
    zero_acc(acc);
    mma_rows<T, RB, 4>(acc, x, Ws, LDW);
#pragma unroll
    for (int rb = 0; rb < RB; rb++)
#pragma unroll
      for (int cb = 0; cb < 4; cb++)
#pragma unroll
        for (int e = 0; e < 4; e++) gate[rb][4 * cc + cb][e] = sigmoidf_(acc[rb][cb][e]);
  }
  // LN_out rows as the B operand, p_out chunks
#pragma unroll
  for (int rb = 0; rb < RB; rb++) RG<T>::load_row(x[rb], Ts + (wave * 16 * RB + 16 * rb + (l & 15)) * LDW, g);
  f4 y[RB][8];
#pragma unroll
  for (int cc = 0; cc < 2; cc++) {
    __syncthreads();
    lds_rows<T>(Ws, LDW, 64, D, [&](int r) { return w_po + (int64_t)(64 * cc + r) * D; });
    __syncthreads();
    f4 acc[RB][4];
    zero_acc(acc);
    mma_rows<T, RB, 4>(acc, x, Ws, LDW);
#pragma unroll
    for (int rb = 0; rb < RB; rb++)
#pragma unroll
      for (int cb = 0; cb < 4; cb++) y[rb][4 * cc + cb] = acc[rb][cb] * gate[rb][4 * cc + cb];
  }
  resid_ln_rows<T, RB>(y, [&](int rb) -> int64_t { return jpos[rb] < N ? i * N + jpos[rb] : -1; }, z, accumulate, lnw,
                       lnb, eps_next, xn_next);
}

// ---------------------------------------------------------------- triangle attention projection
// grid: ceil(N^2 / TM) position tiles; M = 4*H*C + H output channels in 64-channel chunks.
template <typename T>
__global__ __launch_bounds__(256) void triattn_proj_k(const T* __restrict__ xn, const T* __restrict__ w, int trans,
                                                      float q_scale, float b_scale, T* __restrict__ qkg,
                                                      T* __restrict__ vt, T* __restrict__ tb, int64_t N, int64_t ldk,
                                                      int H, int C) {
  constexpr int RB = RowBlocks<T>::v, TM = 64 * RB, STEPS = RG<T>::STEPS, LDW = ldw_of<T>();
  __shared__ LDS_ALIGN T Ws[64 * LDW];
  const int64_t NN = N * N;
  const int64_t p0 = (int64_t)blockIdx.x * TM;
  const int HC = H * C, M = 4 * HC + H;
  const int wave = threadIdx.x >> 6, l = threadIdx.x & 63, g = l >> 4;

  typename RG<T>::frag x[RB][STEPS];
  int64_t pos[RB];
#pragma unroll
  for (int rb = 0; rb < RB; rb++) {
    pos[rb] = p0 + wave * 16 * RB + 16 * rb + (l & 15);
    int64_t p = pos[rb] < NN ? pos[rb] : NN - 1;
    if (trans) { const int64_t a = p / N, b = p - a * N; p = b * N + a; }
    RG<T>::load_row(x[rb], xn + p * D, g);
  }
  for (int c0 = 0; c0 < M; c0 += 64) {
    __syncthreads();
    lds_rows<T>(Ws, LDW, 64, D, [&](int r) -> const T* { return c0 + r < M ? w + (int64_t)(c0 + r) * D : nullptr; });
    __syncthreads();
    f4 acc[RB][4];
    zero_acc(acc);
    mma_rows<T, RB, 4>(acc, x, Ws, LDW);
    const int plane4 = c0 / HC;  // 0 q, 1 k, 2 v, 3 g, 4 tri bias (HC % 64 == 0: chunks never straddle)
    const float sc = plane4 == 0 ? q_scale : (plane4 == 4 ? b_scale : 1.0f);
#pragma unroll
    for (int rb = 0; rb < RB; rb++) {
      const int64_t p = pos[rb];
      if (p >= NN) continue;
      const int64_t pi = p / N, pj = p - pi * N;
#pragma unroll
      for (int cb = 0; cb < 4; cb++) {
        const int col = c0 + 16 * cb + 4 * g;  // 4 consecutive channels col .. col+3
        const f4 v = acc[rb][cb] * sc;
        if (plane4 == 0 || plane4 == 1 || plane4 == 3) {
          const int within = col - plane4 * HC;
          const int64_t plane = (int64_t)(plane4 == 3 ? 2 : plane4) * H + within / C;
          st4(qkg + (plane * NN + p) * C + (within % C), v);
        } else if (plane4 == 2) {
          const int within = col - 2 * HC;
          const int hh = within / C, d = within % C;
          T* dst = vt + (((int64_t)hh * N + pi) * C + d) * ldk + pj;
#pragma unroll
          for (int e = 0; e < 4; e++) dst[(int64_t)e * ldk] = from_f<T>(v[e]);
        } else {
#pragma unroll
          for (int e = 0; e < 4; e++) {
            const int hh = col - 4 * HC + e;
            if (hh >= H) continue;
            tb[tb_offset(hh, pi, pj, N, ldk)] = from_f<T>(v[e]);
            if (pj == N - 1)  // finite padding: the MFMA core adds it before masking keys past N
              for (int64_t k = N; k < ldk; k++) tb[tb_offset(hh, pi, k, N, ldk)] = from_f<T>(0.0f);
          }
        }
      }
    }
  }
}

// ---------------------------------------------------------------- linear_o + residual + next LayerNorm
template <typename T>
__global__ __launch_bounds__(256) void linear_resid_ln_k(const T* __restrict__ x_in, const T* __restrict__ w,
                                                         int trans, float* __restrict__ z, int accumulate,
                                                         const float* __restrict__ lnw, const float* __restrict__ lnb,
                                                         float eps, T* __restrict__ xn_next, int64_t N) {
  constexpr int RB = RowBlocks<T>::v, TM = 64 * RB, STEPS = RG<T>::STEPS, LDW = ldw_of<T>();
  __shared__ LDS_ALIGN T Ws[64 * LDW];
  const int64_t NN = N * N;
  const int64_t p0 = (int64_t)blockIdx.x * TM;
  const int wave = threadIdx.x >> 6, l = threadIdx.x & 63, g = l >> 4;
  typename RG<T>::frag x[RB][STEPS];
  int64_t pos[RB];
#pragma unroll
  for (int rb = 0; rb < RB; rb++) {
    pos[rb] = p0 + wave * 16 * RB + 16 * rb + (l & 15);
    RG<T>::load_row(x[rb], x_in + (pos[rb] < NN ? pos[rb] : NN - 1) * D, g);
  }
  f4 y[RB][8];
#pragma unroll
  for (int cc = 0; cc < 2; cc++) {
    __syncthreads();
    lds_rows<T>(Ws, LDW, 64, D, [&](int r) { return w + (int64_t)(64 * cc + r) * D; });
    __syncthreads();
    f4 acc[RB][4];
    zero_acc(acc);
    mma_rows<T, RB, 4>(acc, x, Ws, LDW);
#pragma unroll
    for (int rb = 0; rb < RB; rb++)
#pragma unroll
      for (int cb = 0; cb < 4; cb++) y[rb][4 * cc + cb] = acc[rb][cb];
  }
  resid_ln_rows<T, RB>(y, [&](int rb) -> int64_t {
    int64_t p = pos[rb];
    if (p >= NN) return -1;
    if (trans) { const int64_t a = p / N, b = p - a * N; p = b * N + a; }
    return p;
  }, z, accumulate, lnw, lnb, eps, xn_next);
}

// ---------------------------------------------------------------- transition
// Hidden chunks of HCH units: h1^T, h2^T = fc1/fc2 chunk . xn^T (16-unit blocks), a = silu(h1) * h2 stays in the
// accumulator layout, which is already the B operand layout of out^T += fc3[:, chunk] . a^T (keys of the fp16 MFMA
// permuted as {4g .. 4g+3} u {16+4g .. 16+4g+3} within each 32-unit slice; fp32 steps take unit 4g + s).
template <typename T, int HCH>
__global__ __launch_bounds__(256) void transition_k(const T* __restrict__ xn, const T* __restrict__ w12,
                                                    const T* __restrict__ w3, float* __restrict__ z, int accumulate,
                                                    const float* __restrict__ lnw, const float* __restrict__ lnb,
                                                    float eps, T* __restrict__ xn_next, int64_t rows_total,
                                                    int hidden) {
  constexpr int RB = RowBlocks<T>::v, TM = 64 * RB, STEPS = RG<T>::STEPS, LDW = ldw_of<T>();
  constexpr int LDH = HCH + Pad<T>::v;
  constexpr int HB = HCH / 16;
  __shared__ LDS_ALIGN T W1s[HCH * LDW];
  __shared__ LDS_ALIGN T W2s[HCH * LDW];
  __shared__ LDS_ALIGN T W3s[D * LDH];
  const int64_t r0 = (int64_t)blockIdx.x * TM;
  const int wave = threadIdx.x >> 6, l = threadIdx.x & 63, g = l >> 4;
  typename RG<T>::frag x[RB][STEPS];
  int64_t row[RB];
#pragma unroll
  for (int rb = 0; rb < RB; rb++) {
    row[rb] = r0 + wave * 16 * RB + 16 * rb + (l & 15);
    RG<T>::load_row(x[rb], xn + (row[rb] < rows_total ? row[rb] : rows_total - 1) * D, g);
  }
  f4 out[RB][8];
  zero_acc(out);
  for (int h0 = 0; h0 < hidden; h0 += HCH) {
    __syncthreads();
    lds_rows<T>(W1s, LDW, HCH, D, [&](int r) { return w12 + (int64_t)(h0 + r) * D; });
    lds_rows<T>(W2s, LDW, HCH, D, [&](int r) { return w12 + (int64_t)(hidden + h0 + r) * D; });
    lds_rows<T>(W3s, LDH, D, HCH, [&](int r) { return w3 + (int64_t)r * hidden + h0; });
    __syncthreads();
    f4 a[RB][HB];
#pragma unroll
    for (int hb = 0; hb < HB; hb++) {
      f4 h1[RB][1], h2[RB][1];
      zero_acc(h1);
      zero_acc(h2);
      mma_rows<T, RB, 1>(h1, x, W1s + 16 * hb * LDW, LDW);
      mma_rows<T, RB, 1>(h2, x, W2s + 16 * hb * LDW, LDW);
#pragma unroll
      for (int rb = 0; rb < RB; rb++)
#pragma unroll
        for (int e = 0; e < 4; e++) a[rb][hb][e] = siluf_(h1[rb][0][e]) * h2[rb][0][e];
    }
    if constexpr (sizeof(T) == 2) {
#pragma unroll
      for (int m = 0; m < HB / 2; m++) {
        half8 bf[RB];
#pragma unroll
        for (int rb = 0; rb < RB; rb++)
#pragma unroll
          for (int e = 0; e < 4; e++) {
            bf[rb][e] = (half_t)a[rb][2 * m][e];
            bf[rb][4 + e] = (half_t)a[rb][2 * m + 1][e];
          }
#pragma unroll
        for (int ob = 0; ob < 8; ob++) {
          const T* wr = W3s + (16 * ob + (l & 15)) * LDH + 32 * m + 4 * g;
          const half4 lo = *reinterpret_cast<const half4*>(wr);
          const half4 hi = *reinterpret_cast<const half4*>(wr + 16);
          const half8 af = half8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
#pragma unroll
          for (int rb = 0; rb < RB; rb++)
            out[rb][ob] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af, bf[rb], out[rb][ob], 0, 0, 0);
        }
      }
    } else {
#pragma unroll
      for (int hb = 0; hb < HB; hb++)
#pragma unroll
        for (int s = 0; s < 4; s++)
#pragma unroll
          for (int ob = 0; ob < 8; ob++) {
            const float af = to_f(W3s[(16 * ob + (l & 15)) * LDH + 16 * hb + 4 * g + s]);
#pragma unroll
            for (int rb = 0; rb < RB; rb++)
              out[rb][ob] = __builtin_amdgcn_mfma_f32_16x16x4f32(af, a[rb][hb][s], out[rb][ob], 0, 0, 0);
          }
    }
  }
  resid_ln_rows<T, RB>(out, [&](int rb) -> int64_t { return row[rb] < rows_total ? row[rb] : -1; }, z, accumulate, lnw,
                       lnb, eps, xn_next);
}

}  // namespace

// ---------------------------------------------------------------- launchers

template <typename T>
static hipError_t tm_proj(const void* xn, const void* w, const float* mask, float scale, int incoming, void* ab,
                          int64_t N, int64_t ld, hipStream_t st) {
  constexpr int TM = 64 * RowBlocks<T>::v;
  const dim3 grid((unsigned)(N * ((ld + TM - 1) / TM)));
  trimul_proj_k<T><<<grid, 256, 0, st>>>(static_cast<const T*>(xn), static_cast<const T*>(w), mask, scale, incoming,
                                         static_cast<T*>(ab), N, ld);
  return hipGetLastError();
}

hipError_t launch_trimul_proj(const void* xn, const void* w, const float* mask, float scale, int incoming, void* ab,
                              int dt, int64_t N, int64_t ld, hipStream_t st) {
  return dt == DT_F16 ? tm_proj<half_t>(xn, w, mask, scale, incoming, ab, N, ld, st)
                      : tm_proj<float>(xn, w, mask, scale, incoming, ab, N, ld, st);
}

template <typename T>
static hipError_t tm_tail(const void* o, const float* now, const float* nob, float eps_out, const void* w_po,
                          const void* xn, const void* w_go, float* z, int accumulate, const float* lnw,
                          const float* lnb, float eps_next, void* xn_next, int64_t N, int64_t ld, hipStream_t st) {
  constexpr int TM = 64 * RowBlocks<T>::v;
  const dim3 grid((unsigned)(N * ((ld + TM - 1) / TM)));
  trimul_tail_k<T><<<grid, 256, 0, st>>>(static_cast<const T*>(o), now, nob, eps_out, static_cast<const T*>(w_po),
                                         static_cast<const T*>(xn), static_cast<const T*>(w_go), z, accumulate, lnw,
                                         lnb, eps_next, static_cast<T*>(xn_next), N, ld);
  return hipGetLastError();
}

hipError_t launch_trimul_tail(const void* o, const float* now, const float* nob, float eps_out, const void* w_po,
                              const void* xn, const void* w_go, float* z, int accumulate, const float* lnw,
                              const float* lnb, float eps_next, void* xn_next, int dt, int64_t N, int64_t ld,
                              hipStream_t st) {
  return dt == DT_F16 ? tm_tail<half_t>(o, now, nob, eps_out, w_po, xn, w_go, z, accumulate, lnw, lnb, eps_next,
                                        xn_next, N, ld, st)
                      : tm_tail<float>(o, now, nob, eps_out, w_po, xn, w_go, z, accumulate, lnw, lnb, eps_next,
                                       xn_next, N, ld, st);
}

template <typename T>
static hipError_t ta_proj(const void* xn, const void* w, int trans, float q_scale, float b_scale, void* qkg, void* vt,
                          void* tb, int64_t N, int64_t ldk, int H, int C, hipStream_t st) {
  constexpr int TM = 64 * RowBlocks<T>::v;
  const dim3 grid((unsigned)((N * N + TM - 1) / TM));
  triattn_proj_k<T><<<grid, 256, 0, st>>>(static_cast<const T*>(xn), static_cast<const T*>(w), trans, q_scale,
                                          b_scale, static_cast<T*>(qkg), static_cast<T*>(vt), static_cast<T*>(tb), N,
                                          ldk, H, C);
  return hipGetLastError();
}

hipError_t launch_triattn_proj(const void* xn, const void* w, int trans, float q_scale, float b_scale, void* qkg,
                               void* vt, void* tb, int dt, int64_t N, int64_t ldk, int H, int C, hipStream_t st) {
  return dt == DT_F16 ? ta_proj<half_t>(xn, w, trans, q_scale, b_scale, qkg, vt, tb, N, ldk, H, C, st)
                      : ta_proj<float>(xn, w, trans, q_scale, b_scale, qkg, vt, tb, N, ldk, H, C, st);
}

template <typename T>
static hipError_t lrl(const void* x, const void* w, int trans, float* z, int accumulate, const float* lnw,
                      const float* lnb, float eps, void* xn_next, int64_t N, hipStream_t st) {
  constexpr int TM = 64 * RowBlocks<T>::v;
  const dim3 grid((unsigned)((N * N + TM - 1) / TM));
  linear_resid_ln_k<T><<<grid, 256, 0, st>>>(static_cast<const T*>(x), static_cast<const T*>(w), trans, z, accumulate,
                                             lnw, lnb, eps, static_cast<T*>(xn_next), N);
  return hipGetLastError();
}

hipError_t launch_linear_resid_ln(const void* x, const void* w, int trans, float* z, int accumulate,
                                  const float* lnw, const float* lnb, float eps, void* xn_next, int dt, int64_t N,
                                  hipStream_t st) {
  return dt == DT_F16 ? lrl<half_t>(x, w, trans, z, accumulate, lnw, lnb, eps, xn_next, N, st)
                      : lrl<float>(x, w, trans, z, accumulate, lnw, lnb, eps, xn_next, N, st);
}

template <typename T, int HCH>
static hipError_t trans_t(const void* xn, const void* w12, const void* w3, float* z, int accumulate, const float* lnw,
                          const float* lnb, float eps, void* xn_next, int64_t rows, int hidden, hipStream_t st) {
  if (hidden % HCH) return hipErrorInvalidValue;
  constexpr int TM = 64 * RowBlocks<T>::v;
  const dim3 grid((unsigned)((rows + TM - 1) / TM));
  transition_k<T, HCH><<<grid, 256, 0, st>>>(static_cast<const T*>(xn), static_cast<const T*>(w12),
                                             static_cast<const T*>(w3), z, accumulate, lnw, lnb, eps,
                                             static_cast<T*>(xn_next), rows, hidden);
  return hipGetLastError();
}

hipError_t launch_transition(const void* xn, const void* w12, const void* w3, float* z, int accumulate,
                             const float* lnw, const float* lnb, float eps, void* xn_next, int dt, int64_t rows,
                             int hidden, hipStream_t st) {
  return dt == DT_F16 ? trans_t<half_t, 64>(xn, w12, w3, z, accumulate, lnw, lnb, eps, xn_next, rows, hidden, st)
                      : trans_t<float, 32>(xn, w12, w3, z, accumulate, lnw, lnb, eps, xn_next, rows, hidden, st);
}

}  // namespace bzpf
