// Triangle multiplication contraction: o[c, i, j] = sum_k a[c, i, k] * b[c, j, k], D independent N x N x N "NT"
// GEMMs on MFMA over the channel-major operands written by the projection (bzpf_pair_gemm.hip), which stores the
// incoming direction's operands transposed so that both directions contract the same way.
// Reference behaviour: boltz_mlx/layers/triangular_mult.py:90-93, 172-175 (per-channel matmul),
// kernels_nax2.py:315-407 (contraction kernel).
// Layout: ab is [2D][N][ld] and o is [D][N][ld] with ld = N rounded up to 64 and zero padding in k >= N, so the
// contraction's k loop and the 64-wide position tiles of proj/tail never straddle a row.
#include "bzpf_common.h"
#include "bzpf_kernels.h"

namespace bzpf {

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

}  // namespace bzpf
