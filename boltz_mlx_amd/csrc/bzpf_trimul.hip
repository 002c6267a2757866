// Triangle multiplication (outgoing and incoming) as three kernels:
//   proj     : ab[c, i, k] = (xn W_p[c]) * sigmoid(xn W_g[c]) * mask * scale, channel-major, for the position
//              (i, k) (outgoing) or (k, i) (incoming), so that both directions contract the same way;
//   contract : o[c, i, j] = sum_k a[c, i, k] * b[c, j, k]  (D independent N x N x N "NT" GEMMs on MFMA);
//   tail     : z[i, j] (+)= p_out(LN_out(o[:, i, j])) * sigmoid(g_out(xn[i, j])), then the next LN of z.
// Reference behaviour: boltz_mlx/layers/triangular_mult.py:40-105 (fp32), 107-182 (f16: 2^-K pre-scale of a and
// b, norm_out eps * 2^-4K), kernels_nax2.py:202-304 (channel-major projection), 315-407 (contraction),
// kernels_nax3.py:200-268 (fused tail).
// Layout: ab is [2D][N][ld] and o is [D][N][ld] with ld = N rounded up to 64 and zero padding in k >= N, so the
// contraction's k loop and the 64-wide position tiles of proj/tail never straddle a row.
#include "bzpf_common.h"
#include "bzpf_kernels.h"

namespace bzpf {

constexpr int TM_D = 128;  // pair channel count handled by these kernels

// ---------------------------------------------------------------- projection + gate + mask
// grid: (N * ld / 64 position tiles, 2D / (32 * CPB) channel groups); block 256.
template <typename T, int CPB>
__global__ __launch_bounds__(256) void trimul_proj_kernel(const T* __restrict__ xn, const T* __restrict__ w,
                                                          const float* __restrict__ mask, float scale, int incoming,
                                                          T* __restrict__ ab, int64_t N, int64_t ld) {
  constexpr int D = TM_D, PAD = Pad<T>::v, LDX = D + PAD;
  constexpr int LDO = 64 + PAD;
  __shared__ LDS_ALIGN T Xs[64 * LDX];
  __shared__ LDS_ALIGN T Ws[64 * LDX];
  __shared__ LDS_ALIGN T Os[32 * LDO];
  __shared__ float mk[64];

  const int64_t tiles_per_row = ld / 64;
  const int64_t i = blockIdx.x / tiles_per_row;
  const int64_t k0 = (blockIdx.x - i * tiles_per_row) * 64;
  const int wave = threadIdx.x >> 6, l = threadIdx.x & 63;

  auto src = [&](int r) -> int64_t {
    int64_t k = k0 + r;
    if (k >= N) k = N - 1;  // padding columns: any valid row, the mask zeroes the output
    return incoming ? (k * N + i) : (i * N + k);
  };
  load_rows<T>(Xs, LDX, 64, D, [&](int r) { return xn + src(r) * D; });
  if (threadIdx.x < 64) {
    const int r = threadIdx.x;
    mk[r] = (k0 + r < N) ? mask[src(r)] * scale : 0.0f;
  }

  const int cg0 = blockIdx.y * 32 * CPB;
  for (int cc = 0; cc < CPB; cc++) {
    const int c0 = cg0 + 32 * cc;  // 32 output channels of [a | b]
    __syncthreads();               // Ws / Os reuse
    load_rows<T>(Ws, LDX, 64, D, [&](int r) { return w + (int64_t)(r < 32 ? c0 + r : 2 * D + c0 + r - 32) * D; });
    __syncthreads();
    f4 acc[1][4];
    zero_acc(acc);
    wave_mma<T, 1, 4>(acc, Xs + 16 * wave * LDX, LDX, Ws, LDX, D);
#pragma unroll
    for (int nb = 0; nb < 2; nb++) {
#pragma unroll
      for (int e = 0; e < 4; e++) {
        const int r = 16 * wave + (l >> 4) * 4 + e;
        const int c = 16 * nb + (l & 15);
        const float v = acc[0][nb][e] * sigmoidf_(acc[0][nb + 2][e]) * mk[r];
        Os[c * LDO + r] = from_f<T>(v);
      }
    }
    __syncthreads();
    // 32 channels x 64 positions, each channel row contiguous in ab
    constexpr int VE = Vec16<T>::n;
    for (int e = threadIdx.x; e < 32 * (64 / VE); e += 256) {
      const int c = e / (64 / VE), r = (e - c * (64 / VE)) * VE;
      T* dst = ab + ((int64_t)(c0 + c) * N + i) * ld + k0 + r;
      *reinterpret_cast<U128*>(dst) = *reinterpret_cast<const U128*>(Os + c * LDO + r);
    }
  }
}

// ---------------------------------------------------------------- per-channel contraction
// o[c][i][j] = sum_{k < ld} a[c][i][k] * b[c][j][k]; grid (ceil(N/BT)^2, D); block 256 = 4 waves in 2 x 2, each
// wave a (BT/2) x (BT/2) block of 16x16 MFMA tiles. BK = 32 keys per LDS stage.
template <typename T, int BT>
__global__ __launch_bounds__(256) void trimul_contract_kernel(const T* __restrict__ ab, T* __restrict__ o, int64_t N,
                                                              int64_t ld, int D) {
  constexpr int BK = 32, PAD = Pad<T>::v, LDK = BK + PAD;
  constexpr int WB = BT / 32;  // 16x16 blocks per wave per dimension
  __shared__ LDS_ALIGN T As[BT * LDK];
  __shared__ LDS_ALIGN T Bs[BT * LDK];
  const int64_t tiles = (N + BT - 1) / BT;
  const int64_t ti = blockIdx.x / tiles, tj = blockIdx.x - ti * tiles;
  const int64_t i0 = ti * BT, j0 = tj * BT;
  const int64_t c = blockIdx.y;
  const T* a = ab + c * N * ld;
  const T* b = ab + ((int64_t)D + c) * N * ld;
  const int wave = threadIdx.x >> 6, l = threadIdx.x & 63;
  const int wr = wave >> 1, wc = wave & 1;

  f4 acc[WB][WB];
  zero_acc(acc);
  for (int64_t k0 = 0; k0 < ld; k0 += BK) {
    __syncthreads();
    load_rows<T>(As, LDK, BT, BK, [&](int r) { int64_t ii = i0 + r; if (ii >= N) ii = N - 1; return a + ii * ld + k0; });
    load_rows<T>(Bs, LDK, BT, BK, [&](int r) { int64_t jj = j0 + r; if (jj >= N) jj = N - 1; return b + jj * ld + k0; });
    __syncthreads();
    wave_mma<T, WB, WB>(acc, As + (wr * BT / 2) * LDK, LDK, Bs + (wc * BT / 2) * LDK, LDK, BK);
  }
  T* oc = o + c * N * ld;
#pragma unroll
  for (int mb = 0; mb < WB; mb++)
#pragma unroll
    for (int nb = 0; nb < WB; nb++)
#pragma unroll
      for (int e = 0; e < 4; e++) {
        const int64_t ii = i0 + wr * BT / 2 + 16 * mb + (l >> 4) * 4 + e;
        const int64_t jj = j0 + wc * BT / 2 + 16 * nb + (l & 15);
        if (ii < N && jj < N) oc[ii * ld + jj] = from_f<T>(acc[mb][nb][e]);
      }
}

// ---------------------------------------------------------------- fused tail
// grid: N * ld / 64 position tiles (i, j0 .. j0+63); block 256 (wave w: rows 16w .. 16w+15, all 128 columns).
template <typename T>
__global__ __launch_bounds__(256) void trimul_tail_kernel(const T* __restrict__ o, const float* __restrict__ now,
                                                          const float* __restrict__ nob, float eps_out,
                                                          const T* __restrict__ w_po, const T* __restrict__ xn,
                                                          const T* __restrict__ w_go, float* __restrict__ z,
                                                          int accumulate, const float* __restrict__ lnw,
                                                          const float* __restrict__ lnb, float eps_next,
                                                          T* __restrict__ xn_next, int64_t N, int64_t ld) {
  constexpr int D = TM_D, PAD = Pad<T>::v, LDX = D + PAD, LDY = D + 4;
  // Ts and Xs are contiguous so that the fp32 output staging Ys can reuse them after the GEMMs.
  constexpr int TX_BYTES = 2 * 64 * LDX * (int)sizeof(T);
  constexpr int Y_BYTES = 64 * LDY * 4;
  __shared__ LDS_ALIGN char smem[(TX_BYTES > Y_BYTES ? TX_BYTES : Y_BYTES)];
  __shared__ LDS_ALIGN T Wsh[64 * LDX];
  T* Ts = reinterpret_cast<T*>(smem);
  T* Xs = Ts + 64 * LDX;
  float* Ys = reinterpret_cast<float*>(smem);

  const int64_t tiles_per_row = ld / 64;
  const int64_t i = blockIdx.x / tiles_per_row;
  const int64_t j0 = (blockIdx.x - i * tiles_per_row) * 64;
  const int wave = threadIdx.x >> 6, l = threadIdx.x & 63;
  const int rows = (int)((N - j0) < 64 ? (N - j0) : 64);

  // o tile, transposed into Ts[r][c]: each channel row of o is 64 contiguous positions
  {
    constexpr int VE = Vec16<T>::n;
    for (int e = threadIdx.x; e < D * (64 / VE); e += 256) {
      const int c = e / (64 / VE), r = (e - c * (64 / VE)) * VE;
      U128 v = *reinterpret_cast<const U128*>(o + ((int64_t)c * N + i) * ld + j0 + r);
      const T* vv = reinterpret_cast<const T*>(&v);
#pragma unroll
      for (int u = 0; u < VE; u++) Ts[(r + u) * LDX + c] = vv[u];
    }
  }
  load_rows<T>(Xs, LDX, 64, D, [&](int r) { int64_t j = j0 + r; if (j >= N) j = N - 1; return xn + (i * N + j) * D; });
  __syncthreads();
  // LN_out over the 128 channels of each position (4 threads per row)
  {
    const int r = threadIdx.x >> 2, q = threadIdx.x & 3;
    T* tr = Ts + r * LDX + q * 32;
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
  // gates: G = Xs W_go^T, two 64-column chunks
  f4 g[1][8], p[1][8];
  zero_acc(g);
  zero_acc(p);
  for (int cc = 0; cc < 2; cc++) {
    __syncthreads();
    load_rows<T>(Wsh, LDX, 64, D, [&](int r) { return w_go + (int64_t)(64 * cc + r) * D; });
    __syncthreads();
    f4 t4[1][4];
    zero_acc(t4);
    wave_mma<T, 1, 4>(t4, Xs + 16 * wave * LDX, LDX, Wsh, LDX, D);
#pragma unroll
    for (int nb = 0; nb < 4; nb++) g[0][4 * cc + nb] = t4[0][nb];
  }
  for (int cc = 0; cc < 2; cc++) {
    __syncthreads();
    load_rows<T>(Wsh, LDX, 64, D, [&](int r) { return w_po + (int64_t)(64 * cc + r) * D; });
    __syncthreads();
    f4 t4[1][4];
    zero_acc(t4);
    wave_mma<T, 1, 4>(t4, Ts + 16 * wave * LDX, LDX, Wsh, LDX, D);
#pragma unroll
    for (int nb = 0; nb < 4; nb++) p[0][4 * cc + nb] = t4[0][nb];
  }
  __syncthreads();  // Ts / Xs are overwritten by Ys below
#pragma unroll
  for (int nb = 0; nb < 8; nb++)
#pragma unroll
    for (int e = 0; e < 4; e++) {
      const int r = 16 * wave + (l >> 4) * 4 + e, c = 16 * nb + (l & 15);
      Ys[r * LDY + c] = p[0][nb][e] * sigmoidf_(g[0][nb][e]);
    }
  __syncthreads();
  resid_ln_epilogue<T>(Ys, LDY, rows, [&](int r) -> int64_t { return i * N + j0 + r; }, z, accumulate, lnw, lnb,
                       eps_next, xn_next);
}

template <typename T>
static hipError_t proj_t(const void* xn, const void* w, const float* mask, float scale, int incoming, void* ab,
                         int64_t N, int64_t ld, hipStream_t st) {
  constexpr int CPB = 2;
  const dim3 grid((unsigned)(N * ld / 64), (unsigned)(2 * TM_D / (32 * CPB)));
  trimul_proj_kernel<T, CPB><<<grid, 256, 0, st>>>(static_cast<const T*>(xn), static_cast<const T*>(w), mask, scale,
                                                   incoming, static_cast<T*>(ab), N, ld);
  return hipGetLastError();
}

hipError_t launch_trimul_proj(const void* xn, const void* w, const float* mask, float scale, int incoming, void* ab,
                              int dt, int64_t N, int64_t ld, hipStream_t st) {
  return dt == DT_F16 ? proj_t<half_t>(xn, w, mask, scale, incoming, ab, N, ld, st)
                      : proj_t<float>(xn, w, mask, scale, incoming, ab, N, ld, st);
}

template <typename T>
static hipError_t contract_t(const void* ab, void* o, int64_t N, int64_t ld, int D, hipStream_t st) {
  constexpr int BT = 64;
  const int64_t tiles = (N + BT - 1) / BT;
  const dim3 grid((unsigned)(tiles * tiles), (unsigned)D);
  trimul_contract_kernel<T, BT><<<grid, 256, 0, st>>>(static_cast<const T*>(ab), static_cast<T*>(o), N, ld, D);
  return hipGetLastError();
}

hipError_t launch_trimul_contract(const void* ab, void* o, int dt, int64_t N, int64_t ld, int D, hipStream_t st) {
  return dt == DT_F16 ? contract_t<half_t>(ab, o, N, ld, D, st) : contract_t<float>(ab, o, N, ld, D, st);
}

template <typename T>
static hipError_t tail_t(const void* o, const float* now, const float* nob, float eps_out, const void* w_po,
                         const void* xn, const void* w_go, float* z, int accumulate, const float* lnw,
                         const float* lnb, float eps_next, void* xn_next, int64_t N, int64_t ld, hipStream_t st) {
  const dim3 grid((unsigned)(N * ld / 64));
  trimul_tail_kernel<T><<<grid, 256, 0, st>>>(static_cast<const T*>(o), now, nob, eps_out, static_cast<const T*>(w_po),
                                              static_cast<const T*>(xn), static_cast<const T*>(w_go), z, accumulate,
                                              lnw, lnb, eps_next, static_cast<T*>(xn_next), N, ld);
  return hipGetLastError();
}

hipError_t launch_trimul_tail(const void* o, const float* now, const float* nob, float eps_out, const void* w_po,
                              const void* xn, const void* w_go, float* z, int accumulate, const float* lnw,
                              const float* lnb, float eps_next, void* xn_next, int dt, int64_t N, int64_t ld,
                              hipStream_t st) {
  return dt == DT_F16 ? tail_t<half_t>(o, now, nob, eps_out, w_po, xn, w_go, z, accumulate, lnw, lnb, eps_next,
                                       xn_next, N, ld, st)
                      : tail_t<float>(o, now, nob, eps_out, w_po, xn, w_go, z, accumulate, lnw, lnb, eps_next,
                                      xn_next, N, ld, st);
}

}  // namespace bzpf
