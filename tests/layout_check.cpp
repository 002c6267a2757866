// Host-side check of the kernels' index maps and 32-bit buffer ranges (boltz_mlx_amd/csrc/bzpf_layout.h), built
// with g++ by tests/test_host_layouts.py: no GPU, no HIP. Exports:
//   lc_tb_offsets(N, H, out): tb_offset(h, j, k) for h < H, j < N, k < N in [H][N][N] order;
//   lc_check(report, cap):    every check below; returns the number of failures and writes one line per check.
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include <algorithm>
#include <string>
#include <vector>

#include "bzpf_layout.h"

using namespace bzpf;

extern "C" void lc_tb_offsets(int64_t N, int H, int64_t* out) {
  const int64_t ldk = row_pitch(N);
  for (int64_t h = 0; h < H; h++)
    for (int64_t j = 0; j < N; j++)
      for (int64_t k = 0; k < N; k++) out[(h * N + j) * N + k] = tb_offset(h, j, k, N, ldk);
}

namespace {

struct Report {
  std::string text;
  int failures = 0;
  void line(bool ok, const std::string& what) {
    text += (ok ? "ok   " : "FAIL ") + what + "\n";
    if (!ok) failures++;
  }
};

// tb_offset over the padded index space (h < H, j < 32 * ceil(N / 32), k < row_pitch(N)) is a bijection onto
// [0, tri_bias_numel): every slot is hit exactly once.
bool tb_bijective(int64_t N, int H) {
  const int64_t ldk = row_pitch(N), jp = (N + 31) / 32 * 32, numel = tri_bias_numel(N, H);
  if (numel != (int64_t)H * jp * ldk) return false;
  std::vector<uint8_t> seen((size_t)numel, 0);
  for (int64_t h = 0; h < H; h++)
    for (int64_t j = 0; j < jp; j++)
      for (int64_t k = 0; k < ldk; k++) {
        const int64_t o = tb_offset(h, j, k, N, ldk);
        if (o < 0 || o >= numel || seen[(size_t)o]) return false;
        seen[(size_t)o] = 1;
      }
  return true;
}

// A lane's 32 bias values of one (32-query tile, 64-key block) are four 16-byte runs, and each run is contiguous
// across the 64 lanes of the wave (lane l at 16 l within a 1 KB piece): the core's four loads per block.
bool tb_fragment_runs(int64_t N) {
  const int64_t ldk = row_pitch(N);
  for (int64_t jt = 0; jt < (N + 31) / 32; jt++)
    for (int64_t kb = 0; kb < ldk / 64; kb++) {
      const int64_t base = tb_offset(0, 32 * jt, 64 * kb, N, ldk);
      for (int l = 0; l < 64; l++) {
        const int64_t q = l & 31, hl = l >> 5;
        for (int x = 0; x < 32; x++) {  // element x = 16 kt + 4 p + e: key 32 kt + 8 p + 4 hl + e
          const int64_t key = 64 * kb + 32 * (x >> 4) + 8 * ((x >> 2) & 3) + 4 * hl + (x & 3);
          const int64_t want = base + 512 * (x >> 3) + 8 * l + (x & 7);
          if (tb_offset(0, 32 * jt + q, key, N, ldk) != want) return false;
        }
      }
    }
  return true;
}

// The contraction's swizzle: for every row, chunk -> chunk ^ ct_swz(row) permutes the row's CPR chunks; a fragment
// read (16 lanes on 16 consecutive rows, starting at a multiple of 16, at one logical chunk c) touches 16 different
// 16-byte bank groups of the 256-byte LDS bank cycle, for every c.
template <int BK>
bool swizzle_ok(std::string* why) {
  constexpr int ROWB = BK * 2, CPR = ROWB / 16;
  for (int row = 0; row < 4096; row++) {
    const int s = ct_swz<BK>(row);
    if (s < 0 || s >= CPR) {
      *why = "swizzle out of range";
      return false;
    }
  }
  for (int base = 0; base < 4096; base += 16)
    for (int c = 0; c < CPR; c++) {
      uint32_t groups = 0;
      for (int r = 0; r < 16; r++) {
        const int row = base + r;
        const int64_t addr = (int64_t)row * ROWB + 16 * (c ^ ct_swz<BK>(row));
        groups |= 1u << ((addr / 16) % 16);
      }
      if (groups != 0xffffu) {
        *why = "bank conflict at rows " + std::to_string(base) + ", chunk " + std::to_string(c);
        return false;
      }
    }
  return true;
}

std::string range_str(const BufRange& r) {
  char b[96];
  snprintf(b, sizeof b, "extent %lld, max offset %lld", (long long)r.extent, (long long)r.max_offset);
  return b;
}

}  // namespace

extern "C" int lc_check(char* out, int cap) {
  Report rep;
  for (int64_t N : {1, 2, 31, 32, 33, 63, 64, 65, 100, 130, 257}) {
    for (int H : {1, 3, 4}) rep.line(tb_bijective(N, H), "tb_offset bijective N=" + std::to_string(N) + " H=" +
                                                             std::to_string(H));
    rep.line(tb_fragment_runs(N), "tb_offset fragment runs N=" + std::to_string(N));
  }
  {
    std::string why;
    rep.line(swizzle_ok<64>(&why), "ct_swz<64> bijective, conflict-free " + why);
    why.clear();
    rep.line(swizzle_ok<32>(&why), "ct_swz<32> bijective, conflict-free " + why);
  }
  // The attention core at its launcher's limits (N <= 32767; the mask row's extent below 2^31 for strided masks).
  for (int64_t N : {1, 64, 1000, 32767}) {
    const int64_t ldk = row_pitch(N), nblk = (N + CORE_BK - 1) / CORE_BK;
    for (int64_t sk : {(int64_t)1, N}) {
      if (!core_shape_ok(N, ldk, 32, sk)) {
        // a mask stride the launcher refuses: its extent would not fit
        rep.line(core_m_extent(N, sk) > 0x7fffffffLL, "core refuses N=" + std::to_string(N) + " mask_sk=" +
                                                          std::to_string(sk) + " only for a mask extent >= 2^31");
        continue;
      }
      int64_t k_lane = 0, v_lane = 0, b_lane = 0, m_lane = 0;
      for (int t = 0; t < 256; t++) {
        k_lane = std::max<int64_t>(k_lane, core_k_lane(t, 32));
        v_lane = std::max<int64_t>(v_lane, core_v_lane(t, ldk));
      }
      for (int v = 0; v < 4; v++)
        for (int l = 0; l < 64; l++) b_lane = std::max<int64_t>(b_lane, core_b_lane(v, l));
      for (int l = 0; l < 64; l++) m_lane = std::max<int64_t>(m_lane, core_m_lane(l, sk));
      const int kb = (int)(nblk - 1);
      const BufRange ranges[4] = {{core_k_extent(N, 32), k_lane + core_k_block(kb, 32)},
                                  {core_v_extent(ldk, 32), v_lane + core_v_block(kb)},
                                  {core_b_extent(ldk), b_lane + core_b_block(kb)},
                                  {core_m_extent(N, sk), m_lane + core_m_block(kb, sk)}};
      const char* names[4] = {"K", "V^T", "bias", "mask"};
      for (int i = 0; i < 4; i++)
        rep.line(fits_int(ranges[i]), std::string("core ") + names[i] + " N=" + std::to_string(N) + " mask_sk=" +
                                        std::to_string(sk) + ": " + range_str(ranges[i]));
      // the int-valued offset helpers must not have wrapped: the same offsets in 64 bits
      rep.line((int64_t)kb * CORE_BK * 32 * 2 == core_k_block(kb, 32) &&
                   (int64_t)kb * CORE_BK * sk * 4 == core_m_block(kb, sk) && (int64_t)63 * sk * 4 == core_m_lane(63, sk) &&
                   (31 * ldk + 56) * 2 == core_v_lane(255, ldk),
               "core int offsets without overflow N=" + std::to_string(N) + " mask_sk=" + std::to_string(sk));
    }
    rep.line(!core_shape_ok(32768, row_pitch(32768), 32, 1), "core refuses N=32768");
  }
  // The contraction: the largest N its launcher accepts, and one past it.
  {
    int64_t nmax = 0;
    for (int64_t N = 1; N <= 65535; N++)
      if (contract_shape_ok(N, row_pitch(N))) nmax = N;
    const BufRange r = {contract_extent(nmax, row_pitch(nmax)), contract_max_offset(nmax, row_pitch(nmax))};
    rep.line(nmax >= 32767 && fits_int(r), "contraction at its largest N=" + std::to_string(nmax) + ": " +
                                             range_str(r));
    for (int64_t N : {1, 400, 800, 1000})
      rep.line(fits_int({contract_extent(N, row_pitch(N)), contract_max_offset(N, row_pitch(N))}),
               "contraction N=" + std::to_string(N));
  }
  // The fp16 sequence attention: N at its limit with the widest accepted row pitch, and the model's shapes.
  for (int64_t N : {4, 400, 1000, 32764}) {
    int64_t ld = 8;
    for (int64_t cand = 8; cand <= 16 * 64 * 4; cand += 8)
      if (seqattn_shape_ok(N, cand)) ld = cand;
    if (!seqattn_shape_ok(N, ld)) {
      rep.line(false, "seq attention accepts no row pitch at N=" + std::to_string(N));
      continue;
    }
    for (int hd : {16, 24, 32, 48, 64}) {
      if (hd > ld) continue;
      const BufRange kv = {seqattn_kv_extent(N, ld, hd), seqattn_kv_max_offset(N, ld, hd)};
      const BufRange b = {seqattn_bias_extent(N), seqattn_bias_max_offset(N)};
      rep.line(fits_int(kv) && fits_int(b), "seq attention N=" + std::to_string(N) + " ld_in=" + std::to_string(ld) +
                                            " hd=" + std::to_string(hd) + ": K/V " + range_str(kv) + "; bias " +
                                            range_str(b));
    }
  }
  rep.line(!seqattn_shape_ok(32768, 8), "seq attention refuses N=32768");
  const int n = (int)std::min<size_t>(rep.text.size(), (size_t)(cap - 1));
  memcpy(out, rep.text.data(), (size_t)n);
  out[n] = 0;
  return rep.failures;
}
