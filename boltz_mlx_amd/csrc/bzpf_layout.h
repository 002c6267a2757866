// Index maps and 32-bit buffer ranges of the kernels, in one header that needs no HIP: the kernels and their
// launchers use these functions, and the host build of tests/layout_check.cpp (g++) checks them on the CPU (the
// fragment-ordered triangle-bias layout is a bijection, the contraction's LDS swizzle is bijective and free of bank
// conflicts, and every buffer resource's extent and offsets fit 32 bits at the launchers' size limits).
#pragma once

#include <stdint.h>

#if defined(__HIPCC__)
#define BZPF_HD __host__ __device__
#else
#define BZPF_HD
#endif

namespace bzpf {

// Row pitch of the padded pair rows (ab, o, V^T, the triangle bias): N rounded up to 64.
BZPF_HD inline int64_t row_pitch(int64_t N) { return (N + 63) / 64 * 64; }

// Triangle-bias layout: element (head h, query j, key k) of the [H][N][N] bias, stored in the order the MFMA
// attention core consumes it (the accumulator layout of v_mfma_f32_32x32x16_f16). For a 32-query tile jt and a
// 64-key block kb, lane l = 32*hl + q of a wave owns the 32 values of query 32*jt + q at keys
// 64*kb + 32*kt + 8*p + 4*hl + e (kt < 2, p < 4, e < 4); element x = 16*kt + 4*p + e of lane l sits at
// 512*(x/8) + 8*l + x%8 of the block's 2048, so each of the lane's four 16-byte loads is one contiguous 1 KB across
// the wave (8 whole cache lines). ldk = row_pitch(N); 4 consecutive keys 4m .. 4m + 3 are contiguous.
BZPF_HD inline int64_t tb_offset(int64_t h, int64_t j, int64_t k, int64_t N, int64_t ldk) {
  const int64_t njt = (N + 31) / 32, nkb = ldk / 64;
  const int64_t jt = j >> 5, q = j & 31, kb = k >> 6, kk = k & 63;
  const int64_t kt = kk >> 5, p = (kk >> 3) & 3, hl = (kk >> 2) & 1, e = kk & 3;
  const int64_t x = kt * 16 + p * 4 + e;
  return ((h * njt + jt) * nkb + kb) * 2048 + (x >> 3) * 512 + (hl * 32 + q) * 8 + (x & 7);
}
// Elements of the triangle-bias buffer: H planes of (N rounded up to 32) queries x ldk keys.
BZPF_HD inline int64_t tri_bias_numel(int64_t N, int64_t H) { return H * ((N + 31) / 32) * 32 * row_pitch(N); }

// The contraction's LDS rows: a stage row of BK fp16 values is CPR = BK / 8 chunks of 16 bytes, and LDS chunk p of
// row R holds the row's logical chunk p ^ ct_swz(R), so the fragment reads (16 lanes on 16 consecutive rows at one
// logical chunk) meet 16 different 16-byte bank groups.
template <int BK>
BZPF_HD inline int ct_swz(int row) {
  if constexpr (BK == 64) return (row & 7) ^ ((row >> 3) & 1);  // 8 chunks of a 128-byte row
  else return ((row >> 1) & 3) ^ ((row >> 3) & 1);                // 4 chunks of a 64-byte row
}

// A raw buffer resource covers `extent` bytes from its base (the num_records field, passed as an int); a load's byte
// offset is its lane offset plus its scalar offset (offsets at or past the extent read as zero, which the kernels
// use for padding). The kernels form both in int arithmetic, so extent and largest offset must stay below 2^31.
struct BufRange {
  int64_t extent;
  int64_t max_offset;  // largest lane offset + scalar offset a kernel issues
};
BZPF_HD inline bool fits_int(const BufRange& r) {
  return r.extent >= 0 && r.extent <= 0x7fffffffLL && r.max_offset >= 0 && r.max_offset <= 0x7fffffffLL;
}

// ---- the fp16 attention core (bzpf_triattn_mfma.hip), per (head, row), 64-key blocks, 256 threads.
// K rows [N][C] (thread t stages key t / 4, channels 8 (t % 4) .. + 7), V^T rows [C][ldk] (channel t / 8, keys
// 8 (t % 8) .. + 7), the bias blocks of the workgroup's 32-query tile (nkb blocks of 4 KB; lane l reads 16 bytes at
// 1024 v + 16 l, v < 4) and the mask row (key kb * 64 + l at stride mask_sk floats).
constexpr int CORE_BK = 64;
BZPF_HD inline int core_k_lane(int t, int C) { return ((t >> 2) * C + (t & 3) * 8) * 2; }
BZPF_HD inline int core_k_block(int kb, int C) { return kb * CORE_BK * C * 2; }
BZPF_HD inline int core_v_lane(int t, int64_t ldk) { return (int)(((t >> 3) * ldk + (t & 7) * 8) * 2); }
BZPF_HD inline int core_v_block(int kb) { return kb * CORE_BK * 2; }
BZPF_HD inline int core_b_lane(int v, int l) { return 1024 * v + 16 * l; }
BZPF_HD inline int core_b_block(int kb) { return kb * 4096; }
BZPF_HD inline int core_m_lane(int l, int64_t mask_sk) { return (int)(l * mask_sk * 4); }
BZPF_HD inline int core_m_block(int kb, int64_t mask_sk) { return (int)(kb * CORE_BK * mask_sk * 4); }
BZPF_HD inline int64_t core_k_extent(int64_t N, int C) { return N * C * 2; }
BZPF_HD inline int64_t core_v_extent(int64_t ldk, int C) { return C * ldk * 2; }
BZPF_HD inline int64_t core_b_extent(int64_t ldk) { return ldk / 64 * 4096; }
BZPF_HD inline int64_t core_m_extent(int64_t N, int64_t mask_sk) { return (N - 1) * mask_sk * 4 + 4; }
// the launcher's limits (32-bit offsets over a row's mask, K, V^T and bias)
BZPF_HD inline bool core_shape_ok(int64_t N, int64_t ldk, int C, int64_t mask_sk) {
  return C == 32 && ldk % 64 == 0 && ldk >= N && N >= 1 && N <= 32767 && mask_sk >= 1 &&
         core_m_extent(N, mask_sk) <= 0x7fffffffLL;
}

// ---- the fp16 contraction (bzpf_trimul.hip): per channel, rows of ld fp16 values; a load's lane offset holds the
// row (rows of a 256-row tile, past N reading as zero) and its 16-byte chunk, the scalar offset the 64-element stage.
BZPF_HD inline int64_t contract_extent(int64_t N, int64_t ld) { return N * ld * 2; }
BZPF_HD inline bool contract_shape_ok(int64_t N, int64_t ld) { return N >= 1 && 2 * N * ld < (1LL << 31); }
// the largest offset: the last row of the last 256-row tile, its last chunk, the last stage
BZPF_HD inline int64_t contract_max_offset(int64_t N, int64_t ld) {
  const int64_t rows = (N + 255) / 256 * 256;
  return ((rows - 1) * ld + 56) * 2 + (ld - 64) * 2;
}

// ---- the fp16 sequence attention (bzpf_seqattn_mfma.hip), per (sample, head): K and V rows of pitch ld_in (keys
// past N read as zero), the bias plane [N][N], the mask row [N].
BZPF_HD inline int64_t seqattn_kv_extent(int64_t N, int64_t ld_in, int hd) { return ((N - 1) * ld_in + hd) * 2; }
BZPF_HD inline int64_t seqattn_bias_extent(int64_t N) { return N * N * 2; }
BZPF_HD inline bool seqattn_shape_ok(int64_t N, int64_t ld_in) {
  return N >= 1 && N <= 32767 && N % 4 == 0 && ld_in % 8 == 0 && (N + 64) * ld_in * 2 <= 0x7fffffffLL &&
         N * N * 2 <= 0x7fffffffLL;
}
// the largest K / V offset: the last staged row of the last 64-key block (a block offset rides in the lane
// offset), its last 16-byte vector; the bias: the last query row's last 8-byte piece of the last block
BZPF_HD inline int64_t seqattn_kv_max_offset(int64_t N, int64_t ld_in, int hd) {
  const int64_t blocks = (N + 63) / 64;
  return ((blocks * 64 - 1) * ld_in + hd - 8) * 2;
}
BZPF_HD inline int64_t seqattn_bias_max_offset(int64_t N) {
  const int64_t blocks = (N + 63) / 64;
  return ((N - 1) * N + 4) * 2 + (blocks - 1) * 64 * 2 + (32 + 24) * 2;
}

}  // namespace bzpf
