// Shared device helpers for the bzpf gfx950 kernels: storage types, MFMA fragment traits, LDS tile copies and wave
// reductions.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "bzpf_layout.h"

typedef _Float16 half_t;
typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef float f2 __attribute__((ext_vector_type(2)));
typedef float f16x __attribute__((ext_vector_type(16)));  // accumulator of one 32 x 32 MFMA block

#define LDS_ALIGN __attribute__((aligned(16)))

namespace bzpf {

constexpr int WG = 256;  // threads per workgroup (4 waves of 64)

__device__ __forceinline__ float to_f(float x) { return x; }
__device__ __forceinline__ float to_f(half_t x) { return (float)x; }
template <typename T> __device__ __forceinline__ T from_f(float x);
template <> __device__ __forceinline__ float from_f<float>(float x) { return x; }
template <> __device__ __forceinline__ half_t from_f<half_t>(float x) { return (half_t)x; }

// v_rcp_f32 (1 ulp) instead of the IEEE division sequence (11 more VALU instructions per element): these run once per
// hidden unit / gate element, which makes them the bulk of the VALU work of the kernels that use them.
// exp(-x) = inf gives rcp(inf) = 0, so both saturate like the exact forms.
__device__ __forceinline__ float sigmoidf_(float x) { return __builtin_amdgcn_rcpf(1.0f + __expf(-x)); }
__device__ __forceinline__ float siluf_(float x) { return x * __builtin_amdgcn_rcpf(1.0f + __expf(-x)); }

// A wave-uniform pointer the compiler must treat as redefined where this is called. Inside a tile loop it keeps the
// per-lane addresses derived from the pointer (64-bit pairs per lane) from being hoisted out of the loop, where they
// outlive the register budget and spill; recomputing them costs one 64-bit add each per tile.
template <typename P> __device__ __forceinline__ P* opaque_ptr(P* p) {
  asm volatile("" : "+s"(p));
  return p;
}

// One 16x16 output block of D = A * B^T per MFMA, A and B both K-contiguous ("NT").
// Lane l holds A[l%16][k0 + (l/16)*KP .. +KP-1] and B[l%16][same k] (B row = output column);
// the accumulator f4 holds D[(l/16)*4 + i][l%16], i = 0..3 (layouts checked on gfx950).
template <typename T> struct Mfma;
template <> struct Mfma<float> {
  static constexpr int KP = 1;   // K elements per lane per instruction
  static constexpr int KS = 4;   // K per instruction
  typedef float frag;
  __device__ static __forceinline__ frag load(const float* p) { return *p; }
  __device__ static __forceinline__ f4 run(frag a, frag b, f4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
  }
};
template <> struct Mfma<half_t> {
  static constexpr int KP = 8;
  static constexpr int KS = 32;
  typedef half8 frag;
  __device__ static __forceinline__ frag load(const half_t* p) { return *reinterpret_cast<const half8*>(p); }
  __device__ static __forceinline__ f4 run(frag a, frag b, f4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
};

// LDS row padding (elements) that keeps 16-byte fragment reads of 16 consecutive rows conflict-free.
template <typename T> struct Pad { static constexpr int v = 16 / sizeof(T); };

// acc[mb][nb] += A[16 mb .. +15][0:K] * B[16 nb .. +15][0:K]^T, A/B in LDS with leading dims lda/ldb.
template <typename T, int MB, int NB>
__device__ __forceinline__ void wave_mma(f4 (&acc)[MB][NB], const T* As, int lda, const T* Bs, int ldb, int K) {
  const int l = threadIdx.x & 63;
  constexpr int KP = Mfma<T>::KP, KS = Mfma<T>::KS;
  const T* ap = As + (l & 15) * lda + (l >> 4) * KP;
  const T* bp = Bs + (l & 15) * ldb + (l >> 4) * KP;
#pragma unroll 2
  for (int k0 = 0; k0 < K; k0 += KS) {
    typename Mfma<T>::frag a[MB], b[NB];
#pragma unroll
    for (int mb = 0; mb < MB; mb++) a[mb] = Mfma<T>::load(ap + 16 * mb * lda + k0);
#pragma unroll
    for (int nb = 0; nb < NB; nb++) b[nb] = Mfma<T>::load(bp + 16 * nb * ldb + k0);
#pragma unroll
    for (int mb = 0; mb < MB; mb++)
#pragma unroll
      for (int nb = 0; nb < NB; nb++) acc[mb][nb] = Mfma<T>::run(a[mb], b[nb], acc[mb][nb]);
  }
}

template <int MB, int NB>
__device__ __forceinline__ void zero_acc(f4 (&acc)[MB][NB]) {
#pragma unroll
  for (int mb = 0; mb < MB; mb++)
#pragma unroll
    for (int nb = 0; nb < NB; nb++) acc[mb][nb] = f4{0.f, 0.f, 0.f, 0.f};
}

// 16-byte vector of T.
template <typename T> struct Vec16 { static constexpr int n = 16 / sizeof(T); };

struct alignas(16) U128 { uint32_t w[4]; };
typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));

// Copy `rows` rows of K elements (K % Vec16 == 0) from global into LDS [rows][ld]. src_row(r) gives the global
// row pointer; rows >= valid are zero-filled when zero_invalid, else read from src_row as given.
template <typename T, typename RowFn>
__device__ __forceinline__ void load_rows(T* dst, int ld, int rows, int K, RowFn src_row) {
  constexpr int VE = Vec16<T>::n;
  const int per_row = K / VE;
  for (int e = threadIdx.x; e < rows * per_row; e += blockDim.x) {
    const int r = e / per_row, c = (e - r * per_row) * VE;
    const T* s = src_row(r);
    u32x4_t v = u32x4_t{0u, 0u, 0u, 0u};
    if (s) v = *reinterpret_cast<const u32x4_t*>(s + c);
    *reinterpret_cast<u32x4_t*>(dst + r * ld + c) = v;
  }
}

// Sum over groups of G consecutive lanes (G a power of two <= 64).
template <int G>
__device__ __forceinline__ float group_sum(float v) {
#pragma unroll
  for (int o = G / 2; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}
// Reductions over the lanes l, l^16, l^32, l^48 (the 4 lane groups of a wave) with the gfx950 row / half-wave
// swaps: permlane16_swap(x, x) returns the values of rows {2r, 2r+1} of each row pair as (first, second), and
// permlane32_swap(x, x) the values of the two halves of the wave.
__device__ __forceinline__ float xgroups_max(float v) {
  const unsigned u = __float_as_uint(v);
  const auto a = __builtin_amdgcn_permlane16_swap(u, u, false, false);
  const float m = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
  const unsigned w = __float_as_uint(m);
  const auto b = __builtin_amdgcn_permlane32_swap(w, w, false, false);
  return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}
__device__ __forceinline__ float xgroups_sum(float v) {
  const unsigned u = __float_as_uint(v);
  const auto a = __builtin_amdgcn_permlane16_swap(u, u, false, false);
  const float s = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  const unsigned w = __float_as_uint(s);
  const auto b = __builtin_amdgcn_permlane32_swap(w, w, false, false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

template <int G>
__device__ __forceinline__ float group_max(float v) {
#pragma unroll
  for (int o = G / 2; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}

}  // namespace bzpf
