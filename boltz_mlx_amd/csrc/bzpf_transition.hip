// SwiGLU Transition over rows of D = 128: z (+)= fc3(silu(xn fc1^T) * (xn fc2^T)), then the next LayerNorm, in one
// kernel. The hidden activations never leave the workgroup: for each chunk of HCH hidden units the up-projection
// tile is formed on MFMA, gated in fp32, stored to LDS in the storage type and immediately consumed by the
// down-projection, whose 64 x 128 accumulator stays in registers across chunks.
// Reference behaviour: boltz_mlx/layers/transition.py:27-54, 148-154 (fc1 is the SiLU branch), kernels.py:948-1155
// (fused fp32 transition), kernels_nax2.py:54-190 and kernels_nax3.py:713-827 (f16 variant with fused residual and
// next LN).
#include "bzpf_common.h"
#include "bzpf_kernels.h"

namespace bzpf {

// grid: ceil(rows / 64); block 256 (wave w: rows 16w .. 16w+15). w12 = [fc1; fc2] ([2*hidden][128]), w3 = fc3
// ([128][hidden]).
template <typename T, int HCH>
__global__ __launch_bounds__(256) void transition_kernel(const T* __restrict__ xn, const T* __restrict__ w12,
                                                         const T* __restrict__ w3, float* __restrict__ z,
                                                         int accumulate, const float* __restrict__ lnw,
                                                         const float* __restrict__ lnb, float eps,
                                                         T* __restrict__ xn_next, int64_t rows_total, int hidden) {
  constexpr int D = 128, PAD = Pad<T>::v, LDX = D + PAD, LDH = HCH + PAD, LDY = D + 4;
  constexpr int W12_BYTES = 2 * HCH * LDX * (int)sizeof(T), Y_BYTES = 64 * LDY * 4;
  __shared__ LDS_ALIGN T Xs[64 * LDX];
  __shared__ LDS_ALIGN char wsm[W12_BYTES > Y_BYTES ? W12_BYTES : Y_BYTES];  // W1c|W2c, later the fp32 output
  __shared__ LDS_ALIGN T W3s[D * LDH];
  __shared__ LDS_ALIGN T As[64 * LDH];
  T* W1s = reinterpret_cast<T*>(wsm);
  T* W2s = W1s + HCH * LDX;
  float* Ys = reinterpret_cast<float*>(wsm);
  const int64_t r0 = (int64_t)blockIdx.x * 64;
  const int rows = (int)((rows_total - r0) < 64 ? (rows_total - r0) : 64);
  const int wave = threadIdx.x >> 6, l = threadIdx.x & 63;
  load_rows<T>(Xs, LDX, 64, D, [&](int r) { return xn + (r0 + (r < rows ? r : rows - 1)) * D; });
  f4 out[1][8];
  zero_acc(out);
  for (int h0 = 0; h0 < hidden; h0 += HCH) {
    __syncthreads();
    load_rows<T>(W1s, LDX, HCH, D, [&](int r) { return w12 + (int64_t)(h0 + r) * D; });
    load_rows<T>(W2s, LDX, HCH, D, [&](int r) { return w12 + (int64_t)(hidden + h0 + r) * D; });
    load_rows<T>(W3s, LDH, D, HCH, [&](int r) { return w3 + (int64_t)r * hidden + h0; });
    __syncthreads();
    f4 h1[1][HCH / 16], h2[1][HCH / 16];
    zero_acc(h1);
    zero_acc(h2);
    wave_mma<T, 1, HCH / 16>(h1, Xs + 16 * wave * LDX, LDX, W1s, LDX, D);
    wave_mma<T, 1, HCH / 16>(h2, Xs + 16 * wave * LDX, LDX, W2s, LDX, D);
#pragma unroll
    for (int nb = 0; nb < HCH / 16; nb++)
#pragma unroll
      for (int e = 0; e < 4; e++)
        As[(16 * wave + (l >> 4) * 4 + e) * LDH + 16 * nb + (l & 15)] = from_f<T>(siluf_(h1[0][nb][e]) * h2[0][nb][e]);
    __syncthreads();
    wave_mma<T, 1, 8>(out, As + 16 * wave * LDH, LDH, W3s, LDH, HCH);
  }
  __syncthreads();  // W1s/W2s are reused as Ys
#pragma unroll
  for (int nb = 0; nb < 8; nb++)
#pragma unroll
    for (int e = 0; e < 4; e++) Ys[(16 * wave + (l >> 4) * 4 + e) * LDY + 16 * nb + (l & 15)] = out[0][nb][e];
  __syncthreads();
  resid_ln_epilogue<T>(Ys, LDY, rows, [&](int r) -> int64_t { return r0 + r; }, z, accumulate, lnw, lnb, eps,
                       xn_next);
}

template <typename T, int HCH>
static hipError_t trans_t(const void* xn, const void* w12, const void* w3, float* z, int accumulate, const float* lnw,
                          const float* lnb, float eps, void* xn_next, int64_t rows, int hidden, hipStream_t st) {
  if (hidden % HCH) return hipErrorInvalidValue;
  const dim3 grid((unsigned)((rows + 63) / 64));
  transition_kernel<T, HCH><<<grid, 256, 0, st>>>(static_cast<const T*>(xn), static_cast<const T*>(w12),
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
