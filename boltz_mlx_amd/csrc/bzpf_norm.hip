// Narrow-row LayerNorm and fused residual-add + LayerNorm.
// Reference behaviour: boltz_mlx/kernels.py:438-507 (layer_norm: two-pass fp32 statistics, rsqrt, optional
// affine, output cast fused) and kernels.py:1399-1480 (add_ln: z_new = z + y * scale, optional transposed read of
// y, LN(z_new) with optional transposed write).
// Layout: 16 lanes per row, each lane holding D/16 values as 4-element vectors (coalesced 64-byte+ row segments);
// a workgroup of 256 threads covers 16 rows.
#include <algorithm>

#include "bzpf_common.h"
#include "bzpf_kernels.h"

namespace bzpf {

template <typename T> struct V4;
template <> struct V4<float> {
  __device__ static __forceinline__ f4 load(const float* p) { return *reinterpret_cast<const f4*>(p); }
  __device__ static __forceinline__ void store(float* p, f4 v) { *reinterpret_cast<f4*>(p) = v; }
};
template <> struct V4<half_t> {
  __device__ static __forceinline__ f4 load(const half_t* p) {
    half4 h = *reinterpret_cast<const half4*>(p);
    return f4{(float)h[0], (float)h[1], (float)h[2], (float)h[3]};
  }
  __device__ static __forceinline__ void store(half_t* p, f4 v) {
    half4 h = {(half_t)v[0], (half_t)v[1], (half_t)v[2], (half_t)v[3]};
    *reinterpret_cast<half4*>(p) = h;
  }
};

// Row index for the transposed-token option: a row r = i*N + j of a [N, N, D] tensor maps to j*N + i.
__device__ __forceinline__ int64_t trow(int64_t r, int64_t N, int trans) {
  if (!trans) return r;
  const int64_t i = r / N, j = r - i * N;
  return j * N + i;
}

// NV = D / 64 vectors of 4 per lane (D % 64 == 0, D <= 1024).
template <typename TI, typename TO, int NV>
__global__ __launch_bounds__(256) void layernorm_kernel(const TI* __restrict__ x, const float* __restrict__ w,
                                                        const float* __restrict__ b, float eps, TO* __restrict__ y,
                                                        int64_t rows) {
  constexpr int D = NV * 64;
  const int lane = threadIdx.x & 15;
  const int64_t row = (int64_t)blockIdx.x * 16 + (threadIdx.x >> 4);
  if (row >= rows) return;  // 16-lane groups exit together
  const TI* xr = x + row * D;
  f4 v[NV];
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < NV; i++) {
    v[i] = V4<TI>::load(xr + 64 * i + 4 * lane);
    s += v[i][0] + v[i][1] + v[i][2] + v[i][3];
  }
  const float mean = group_sum<16>(s) * (1.0f / D);
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < NV; i++) {
    f4 d = v[i] - mean;
    ss += d[0] * d[0] + d[1] * d[1] + d[2] * d[2] + d[3] * d[3];
  }
  const float rstd = 1.0f / sqrtf(group_sum<16>(ss) * (1.0f / D) + eps);
  TO* yr = y + row * D;
#pragma unroll
  for (int i = 0; i < NV; i++) {
    const int c = 64 * i + 4 * lane;
    f4 o = (v[i] - mean) * rstd;
    if (w) o *= *reinterpret_cast<const f4*>(w + c);
    if (b) o += *reinterpret_cast<const f4*>(b + c);
    V4<TO>::store(yr + c, o);
  }
}

// z[row] = z[row] + y[trow(row, trans_y)] * scale; ln[trow(row, trans_out)] = LN(z[row]).
template <typename TY, typename TO, int NV>
__global__ __launch_bounds__(256) void add_ln_kernel(float* __restrict__ z, const TY* __restrict__ y, float scale,
                                                     int trans_y, const float* __restrict__ w,
                                                     const float* __restrict__ b, float eps, TO* __restrict__ ln,
                                                     int trans_out, int64_t N) {
  constexpr int D = NV * 64;
  const int lane = threadIdx.x & 15;
  const int64_t row = (int64_t)blockIdx.x * 16 + (threadIdx.x >> 4);
  if (row >= N * N) return;
  float* zr = z + row * D;
  const TY* yr = y + trow(row, N, trans_y) * D;
  f4 v[NV];
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < NV; i++) {
    const int c = 64 * i + 4 * lane;
    v[i] = *reinterpret_cast<const f4*>(zr + c) + V4<TY>::load(yr + c) * scale;
    *reinterpret_cast<f4*>(zr + c) = v[i];
    s += v[i][0] + v[i][1] + v[i][2] + v[i][3];
  }
  if (ln == nullptr) return;
  const float mean = group_sum<16>(s) * (1.0f / D);
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < NV; i++) {
    f4 d = v[i] - mean;
    ss += d[0] * d[0] + d[1] * d[1] + d[2] * d[2] + d[3] * d[3];
  }
  const float rstd = 1.0f / sqrtf(group_sum<16>(ss) * (1.0f / D) + eps);
  TO* orow = ln + trow(row, N, trans_out) * D;
#pragma unroll
  for (int i = 0; i < NV; i++) {
    const int c = 64 * i + 4 * lane;
    f4 o = (v[i] - mean) * rstd;
    if (w) o *= *reinterpret_cast<const f4*>(w + c);
    if (b) o += *reinterpret_cast<const f4*>(b + c);
    V4<TO>::store(orow + c, o);
  }
}

template <typename TI, typename TO>
static hipError_t ln_dispatch(const void* x, const float* w, const float* b, float eps, void* y, int64_t rows, int D,
                              hipStream_t st) {
  const dim3 grid((unsigned)((rows + 15) / 16)), block(256);
  const TI* xi = static_cast<const TI*>(x);
  TO* yo = static_cast<TO*>(y);
  switch (D / 64) {
#define BZ_CASE(nv) \
  case nv: layernorm_kernel<TI, TO, nv><<<grid, block, 0, st>>>(xi, w, b, eps, yo, rows); break;
    BZ_CASE(1) BZ_CASE(2) BZ_CASE(3) BZ_CASE(4) BZ_CASE(5) BZ_CASE(6) BZ_CASE(8) BZ_CASE(12) BZ_CASE(16)
#undef BZ_CASE
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_layernorm(const void* x, int x_dt, const float* w, const float* b, float eps, void* y, int y_dt,
                            int64_t rows, int D, hipStream_t st) {
  if (x_dt == DT_F32 && y_dt == DT_F32) return ln_dispatch<float, float>(x, w, b, eps, y, rows, D, st);
  if (x_dt == DT_F32 && y_dt == DT_F16) return ln_dispatch<float, half_t>(x, w, b, eps, y, rows, D, st);
  if (x_dt == DT_F16 && y_dt == DT_F32) return ln_dispatch<half_t, float>(x, w, b, eps, y, rows, D, st);
  if (x_dt == DT_F16 && y_dt == DT_F16) return ln_dispatch<half_t, half_t>(x, w, b, eps, y, rows, D, st);
  return hipErrorInvalidValue;
}

template <typename TY, typename TO>
static hipError_t addln_dispatch(float* z, const void* y, float scale, int trans_y, const float* w, const float* b,
                                 float eps, void* ln, int trans_out, int64_t N, int D, hipStream_t st) {
  const dim3 grid((unsigned)((N * N + 15) / 16)), block(256);
  const TY* yi = static_cast<const TY*>(y);
  TO* lo = static_cast<TO*>(ln);
  switch (D / 64) {
#define BZ_CASE(nv)                                                                                       \
  case nv:                                                                                                \
    add_ln_kernel<TY, TO, nv><<<grid, block, 0, st>>>(z, yi, scale, trans_y, w, b, eps, lo, trans_out, N); \
    break;
    BZ_CASE(1) BZ_CASE(2) BZ_CASE(3) BZ_CASE(4) BZ_CASE(6)
#undef BZ_CASE
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_add_ln(float* z, const void* y, int y_dt, float scale, int trans_y, const float* w, const float* b,
                         float eps, void* ln, int ln_dt, int trans_out, int64_t N, int D, hipStream_t st) {
  if (y_dt == DT_F32 && ln_dt == DT_F32) return addln_dispatch<float, float>(z, y, scale, trans_y, w, b, eps, ln, trans_out, N, D, st);
  if (y_dt == DT_F32 && ln_dt == DT_F16) return addln_dispatch<float, half_t>(z, y, scale, trans_y, w, b, eps, ln, trans_out, N, D, st);
  if (y_dt == DT_F16 && ln_dt == DT_F32) return addln_dispatch<half_t, float>(z, y, scale, trans_y, w, b, eps, ln, trans_out, N, D, st);
  if (y_dt == DT_F16 && ln_dt == DT_F16) return addln_dispatch<half_t, half_t>(z, y, scale, trans_y, w, b, eps, ln, trans_out, N, D, st);
  return hipErrorInvalidValue;
}

// Count of inf / nan elements, added to *count: the fp16 overflow guard's check of the fp32 residual streams
// (reference: kernels.guard_residual / guard_take, boltz_mlx/kernels.py:1262-1282, applied in model.py:176-193).
// A value is non-finite when its exponent field is all ones (integer test, independent of the compiler's
// floating-point assumptions). Grid-stride over 16-byte vectors; one atomic per wave that found any.
template <typename T>
__global__ __launch_bounds__(256) void count_nonfinite_k(const T* __restrict__ x, int64_t n, int* __restrict__ count) {
  constexpr int VEC = 16 / sizeof(T);
  const int64_t nvec = n / VEC;
  const int64_t stride = (int64_t)gridDim.x * 256;
  int c = 0;
  const auto bad32 = [](uint32_t u) { return (u & 0x7f800000u) == 0x7f800000u; };
  const auto bad16 = [](uint32_t u) { return (u & 0x7c00u) == 0x7c00u; };
  for (int64_t v = (int64_t)blockIdx.x * 256 + threadIdx.x; v < nvec; v += stride) {
    const u32x4_t w = *reinterpret_cast<const u32x4_t*>(x + v * VEC);
#pragma unroll
    for (int e = 0; e < 4; e++) {
      if constexpr (sizeof(T) == 4) {
        c += bad32(w[e]);
      } else {
        c += bad16(w[e] & 0xffffu) + bad16(w[e] >> 16);
      }
    }
  }
  if (blockIdx.x == 0) {  // the tail past the last whole vector
    for (int64_t i = nvec * VEC + threadIdx.x; i < n; i += 256) {
      if constexpr (sizeof(T) == 4) {
        c += bad32(__float_as_uint(x[i]));
      } else {
        c += bad16(__builtin_bit_cast(uint16_t, x[i]));
      }
    }
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) c += __shfl_xor(c, o, 64);
  if ((threadIdx.x & 63) == 0 && c > 0) atomicAdd(count, c);
}

hipError_t launch_count_nonfinite(const void* x, int dt, int64_t n, int* count, hipStream_t st) {
  const int64_t vec = dt == DT_F16 ? 8 : 4;
  const int64_t blocks = std::max<int64_t>(1, std::min<int64_t>((n / vec + 255) / 256, 2048));
  if (dt == DT_F16)
    count_nonfinite_k<half_t><<<(unsigned)blocks, 256, 0, st>>>(static_cast<const half_t*>(x), n, count);
  else
    count_nonfinite_k<float><<<(unsigned)blocks, 256, 0, st>>>(static_cast<const float*>(x), n, count);
  return hipGetLastError();
}

}  // namespace bzpf
