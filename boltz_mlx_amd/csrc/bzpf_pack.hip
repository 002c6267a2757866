// Layout kernels of the pair updates at any channel count (the template stack's c_z = 64; the fused kernels in
// bzpf_pair_gemm.hip are built for 128 channels). The projections themselves are bzpf_linear GEMMs whose [N*N, cols]
// outputs these kernels gate, mask and move into the layouts the contraction and the attention core read:
//   trimul_pack      : ab[c][i][k] = P[p][c] * sigmoid(P[p][2D + c]) * mask[p] * scale, p = (i, k) outgoing or (k, i)
//                      incoming, from P = xn [p_in; g_in]^T (boltz_mlx/layers/triangular_mult.py:40-65);
//   channels_to_rows : out[i N + j][c] = o[c][i][j], the contraction output back to position-major rows for norm_out
//                      (triangular_mult.py:93-98);
//   triattn_pack     : q (scaled), k, g planes, v transposed per row and the fragment-ordered triangle bias (scaled)
//                      from P = xn [q; k; v; g; bias]^T, read at (j, i) for the ending node
//                      (boltz_mlx/layers/triangular_attention/attention.py:49-69, 100-104).
// Each workgroup moves one row i and 64 consecutive positions through LDS, so both the position-major reads and the
// channel-major writes are contiguous.
#include "bzpf_common.h"
#include "bzpf_kernels.h"

namespace bzpf {

namespace {

constexpr int PT = 64;  // positions per workgroup
constexpr int PLD = PT + 1;

template <typename T>
__global__ __launch_bounds__(256) void trimul_pack_k(const T* __restrict__ P, const float* __restrict__ mask,
                                                     float scale, int incoming, T* __restrict__ ab, int N, int64_t ld,
                                                     int D) {
  constexpr int CH = 128;  // channels (of the 2D a | b planes) per LDS pass
  __shared__ float sv[CH * PLD];
  const int i = blockIdx.y, k0 = blockIdx.x * PT, D2 = 2 * D;
  for (int c0 = 0; c0 < D2; c0 += CH) {
    const int nc = min(CH, D2 - c0);
    for (int e = threadIdx.x; e < PT * nc; e += 256) {
      const int kk = e / nc, c = e - kk * nc, k = k0 + kk;
      float v = 0.0f;
      if (k < N) {
        const int64_t p = incoming ? (int64_t)k * N + i : (int64_t)i * N + k;
        v = to_f(P[p * 2 * D2 + c0 + c]) * sigmoidf_(to_f(P[p * 2 * D2 + D2 + c0 + c])) * mask[p] * scale;
      }
      sv[c * PLD + kk] = v;
    }
    __syncthreads();
    for (int e = threadIdx.x; e < PT * nc; e += 256) {
      const int c = e / PT, kk = e - c * PT;
      ab[((int64_t)(c0 + c) * N + i) * ld + k0 + kk] = from_f<T>(sv[c * PLD + kk]);
    }
    __syncthreads();
  }
}

template <typename T, typename TO>
__global__ __launch_bounds__(256) void channels_to_rows_k(const T* __restrict__ o, TO* __restrict__ out, int N,
                                                          int64_t ld, int D) {
  extern __shared__ float sv[];  // [D][PLD]
  const int i = blockIdx.y, j0 = blockIdx.x * PT;
  for (int e = threadIdx.x; e < PT * D; e += 256) {
    const int c = e / PT, jj = e - c * PT;
    sv[c * PLD + jj] = to_f(o[((int64_t)c * N + i) * ld + j0 + jj]);
  }
  __syncthreads();
  for (int e = threadIdx.x; e < PT * D; e += 256) {
    const int jj = e / D, c = e - jj * D, j = j0 + jj;
    if (j < N) out[((int64_t)i * N + j) * D + c] = from_f<TO>(sv[c * PLD + jj]);
  }
}

template <typename T>
__global__ __launch_bounds__(256) void triattn_pack_k(const T* __restrict__ P, int trans, float q_scale, float b_scale,
                                                      T* __restrict__ qkg, T* __restrict__ vt, T* __restrict__ tb,
                                                      int N, int64_t ldk, int H, int C) {
  extern __shared__ float sv[];  // [H C + H][PLD]: v channels, then the bias heads
  const int i = blockIdx.y, j0 = blockIdx.x * PT, HC = H * C, W = 4 * HC + H;
  const int64_t NN = (int64_t)N * N;
  for (int e = threadIdx.x; e < PT * W; e += 256) {
    const int jj = e / W, col = e - jj * W, j = j0 + jj;
    const int64_t src = trans ? (int64_t)j * N + i : (int64_t)i * N + j;
    const float x = j < N ? to_f(P[src * W + col]) : 0.0f;
    const int part = col < 4 * HC ? col / HC : 4, within = col - part * HC;
    if (part == 2) {
      sv[within * PLD + jj] = x;
    } else if (part == 4) {
      sv[(HC + within) * PLD + jj] = x * b_scale;
    } else if (j < N) {  // q (plane 0, scaled), k (plane 1), g (plane 2)
      const int h = within / C, c = within - h * C, plane = part == 3 ? 2 : part;
      qkg[((int64_t)(plane * H + h) * NN + (int64_t)i * N + j) * C + c] = from_f<T>(part == 0 ? x * q_scale : x);
    }
  }
  __syncthreads();
  for (int e = threadIdx.x; e < PT * HC; e += 256) {
    const int ch = e / PT, jj = e - ch * PT, h = ch / C, c = ch - h * C;
    vt[(((int64_t)h * N + i) * C + c) * ldk + j0 + jj] = from_f<T>(sv[ch * PLD + jj]);
  }
  for (int e = threadIdx.x; e < PT * H; e += 256) {
    const int h = e / PT, jj = e - h * PT;
    tb[tb_offset(h, i, j0 + jj, N, ldk)] = from_f<T>(sv[(HC + h) * PLD + jj]);
  }
}

}  // namespace

hipError_t launch_trimul_pack(const void* P, const float* mask, float scale, int incoming, void* ab, int dt,
                              int64_t N, int64_t ld, int D, hipStream_t st) {
  if (N < 1 || N > 65535 || ld % PT || ld < N || D < 1 || D > 4096) return hipErrorInvalidValue;
  const dim3 grid((unsigned)(ld / PT), (unsigned)N);
  if (dt == DT_F16)
    trimul_pack_k<half_t><<<grid, 256, 0, st>>>(static_cast<const half_t*>(P), mask, scale, incoming,
                                                  static_cast<half_t*>(ab), (int)N, ld, D);
  else
    trimul_pack_k<float><<<grid, 256, 0, st>>>(static_cast<const float*>(P), mask, scale, incoming,
                                                 static_cast<float*>(ab), (int)N, ld, D);
  return hipGetLastError();
}

hipError_t launch_channels_to_rows(const void* o, int o_dt, void* out, int out_dt, int64_t N, int64_t ld, int D,
                                   hipStream_t st) {
  if (N < 1 || N > 65535 || ld % PT || ld < N || D < 1 || D * PLD * 4 > 65536) return hipErrorInvalidValue;
  const dim3 grid((unsigned)(ld / PT), (unsigned)N);
  const size_t lds = (size_t)D * PLD * sizeof(float);
#define BZ_C2R(T, TO)                                                                                             \
  channels_to_rows_k<T, TO><<<grid, 256, lds, st>>>(static_cast<const T*>(o), static_cast<TO*>(out), (int)N, ld, D)
  if (o_dt == DT_F16) {
    if (out_dt == DT_F16) BZ_C2R(half_t, half_t); else BZ_C2R(half_t, float);
  } else {
    if (out_dt == DT_F16) BZ_C2R(float, half_t); else BZ_C2R(float, float);
  }
#undef BZ_C2R
  return hipGetLastError();
}

hipError_t launch_triattn_pack(const void* P, int trans, float q_scale, float b_scale, void* qkg, void* vt, void* tb,
                               int dt, int64_t N, int64_t ldk, int H, int C, hipStream_t st) {
  if (N < 1 || N > 65535 || ldk % PT || ldk < N || H < 1 || C < 1 || (int64_t)(H * C + H) * PLD * 4 > 65536)
    return hipErrorInvalidValue;
  const dim3 grid((unsigned)(ldk / PT), (unsigned)N);
  const size_t lds = (size_t)(H * C + H) * PLD * sizeof(float);
  if (dt == DT_F16)
    triattn_pack_k<half_t><<<grid, 256, lds, st>>>(static_cast<const half_t*>(P), trans, q_scale, b_scale,
                                                   static_cast<half_t*>(qkg), static_cast<half_t*>(vt),
                                                   static_cast<half_t*>(tb), (int)N, ldk, H, C);
  else
    triattn_pack_k<float><<<grid, 256, lds, st>>>(static_cast<const float*>(P), trans, q_scale, b_scale,
                                                  static_cast<float*>(qkg), static_cast<float*>(vt),
                                                  static_cast<float*>(tb), (int)N, ldk, H, C);
  return hipGetLastError();
}

}  // namespace bzpf
