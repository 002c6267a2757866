// fp32-accurate products on the bf16 matrix cores. Each fp32 operand value is split exactly into three bf16 parts,
// x = x1 + x2 + x3 (x1 the round-to-nearest-even of x, x2 of x - x1, x3 = x - x1 - x2: 8 significant bits each, 24
// together), and a product is taken as the six part products x_a y_b with a + b <= 4, accumulated in fp32 by
// v_mfma_f32_32x32x16_bf16 (exact bf16 products, fp32 sums); the three left out (x2 y3, x3 y2, x3 y3) are below
// 2^-23 of |x y| together. That is the fp32 matrix cores' accuracy at 6 / 16 of their time (the bf16 rate is 16
// times the fp32 one). Operands sit in LDS as three K-contiguous planes (one per part) of KS = 16 bf16 per row.
#pragma once
#include "bzpf_common.h"

namespace bzpf {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

// Two values split at once: part p of both, packed (value 0 in the low half), one v_cvt_pk_bf16_f32 per part.
struct Pair3 {
  uint32_t p[3];
};
__device__ __forceinline__ uint32_t cvt_pair(float a, float b) {
  return __builtin_bit_cast(uint32_t, bf16x2{(__bf16)a, (__bf16)b});
}
__device__ __forceinline__ Pair3 split3_pair(float x0, float x1) {
#pragma clang fp contract(off)  // the parts are of the rounded x0, x1 (no product of the caller fused in)
  Pair3 o;
  o.p[0] = cvt_pair(x0, x1);
  const float r0 = x0 - __uint_as_float(o.p[0] << 16), r1 = x1 - __uint_as_float(o.p[0] & 0xffff0000u);  // exact
  o.p[1] = cvt_pair(r0, r1);
  // exact: at most 8 significant bits are left
  o.p[2] = cvt_pair(r0 - __uint_as_float(o.p[1] << 16), r1 - __uint_as_float(o.p[1] & 0xffff0000u));
  return o;
}

// LDS plane rows: KS = 16 bf16 at a pitch of LDP = 24 (fragment reads of 8 lanes on 8 consecutive rows hit distinct
// banks); PLANE = a plane of 128 rows.
constexpr int KS = 16, LDP = KS + 8, PLANE = 128 * LDP;

// The six part products of one 32 x 32 block for one K-step (smaller ones first).
__device__ __forceinline__ f16x mfma_parts6(const bf16x8 (&a)[3], const bf16x8 (&b)[3], f16x c) {
  c = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[2], b[0], c, 0, 0, 0);
  c = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[1], b[1], c, 0, 0, 0);
  c = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[0], b[2], c, 0, 0, 0);
  c = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[1], b[0], c, 0, 0, 0);
  c = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[0], b[1], c, 0, 0, 0);
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[0], b[0], c, 0, 0, 0);
}

// One stage of a wave's MB x NB blocks: fragments of the three planes (PA / PB bf16 apart) of A rows
// 32 MB wm + 32 bm + r32 and B rows 32 NB wn + 32 bn + r32, k = 8 hl .. 8 hl + 7 (lane (r32, hl)).
template <int MB = 2, int NB = 2, int PA = PLANE, int PB = PLANE>
__device__ __forceinline__ void parts_stage(const __bf16* Ab, const __bf16* Bb, int wm, int wn, int r32, int hl,
                                            f16x (&acc)[MB][NB]) {
  bf16x8 fa[MB][3], fb[NB][3];
#pragma unroll
  for (int bm = 0; bm < MB; bm++)
#pragma unroll
    for (int p = 0; p < 3; p++)
      fa[bm][p] = *reinterpret_cast<const bf16x8*>(Ab + p * PA + (32 * MB * wm + 32 * bm + r32) * LDP + 8 * hl);
#pragma unroll
  for (int bn = 0; bn < NB; bn++)
#pragma unroll
    for (int p = 0; p < 3; p++)
      fb[bn][p] = *reinterpret_cast<const bf16x8*>(Bb + p * PB + (32 * NB * wn + 32 * bn + r32) * LDP + 8 * hl);
#pragma unroll
  for (int bm = 0; bm < MB; bm++)
#pragma unroll
    for (int bn = 0; bn < NB; bn++) acc[bm][bn] = mfma_parts6(fa[bm], fb[bn], acc[bm][bn]);
}

}  // namespace bzpf
