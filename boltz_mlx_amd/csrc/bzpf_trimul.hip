// Triangle multiplication contraction: o[c, i, j] = sum_k a[c, i, k] * b[c, j, k], D independent N x N x N "NT"
// GEMMs on MFMA over the channel-major operands written by the projection (bzpf_pair_gemm.hip), which stores the
// incoming direction's operands transposed so that both directions contract the same way.
// Reference behaviour: boltz_mlx/layers/triangular_mult.py:90-93, 172-175 (per-channel matmul),
// kernels_nax2.py:315-407 (contraction kernel).
// Layout: ab is [2D][N][ld] and o is [D][N][ld] with ld = N rounded up to 64 and zero padding in k >= N, so the
// contraction's k loop and the 64-wide position tiles of proj/tail never straddle a row.
#include "bzpf_common.h"
#include "bzpf_kernels.h"
#include "bzpf_rowgemm.h"

namespace bzpf {

// ---------------------------------------------------------------- per-channel contraction
// o[c][i][j] = sum_{k < ld} a[c][i][k] * b[c][j][k], a = ab[c], b = ab[D + c] (k >= N is zero padding).
// Workgroup: a 128 x 128 tile (i, j) of one channel, 4 waves in 2 x 2, each 64 x 64 = 4 x 4 MFMA blocks. The tile is
// computed transposed, o^T = b a^T (A operand = rows of b, B operand = rows of a), so each lane holds 4 consecutive
// j of one i and stores them as one vector. K advances BK elements per stage through a double-buffered LDS tile;
// the next stage is loaded into registers while the current one computes. Lane group g of a wave reads the
// contiguous k range [g*BK/4, (g+1)*BK/4) of each stage (a permutation of the k sum shared by A and B).
// Tiles are ordered (channel, tile) and dealt to the XCDs in contiguous ranges, so one channel's a and b stay in
// one XCD's L2.
template <typename T>
__global__ __launch_bounds__(256, 2) void trimul_contract_kernel(const T* __restrict__ ab, T* __restrict__ o,
                                                                 int64_t N, int64_t ld, int D, int64_t tiles1,
                                                                 int64_t units, int64_t per_xcd, int nst) {
  constexpr int BT = 128;
  constexpr int BK = sizeof(T) == 2 ? 64 : 32;      // k per stage: 128 bytes of a row
  constexpr int KG = BK / 4;                        // contiguous k per lane group
  constexpr int KP = Mfma<T>::KP;
  constexpr int STEPS = KG / KP;
  constexpr int LDT = BK + 16 / (int)sizeof(T);     // LDS row pitch (elements)
  constexpr int VE = 16 / (int)sizeof(T);           // elements per 16-byte vector
  constexpr int VPR = BK / VE;                      // vectors per row per stage (8)
  constexpr int LOADS = 2 * BT * VPR / 256;         // 16-byte vectors per thread per stage (8)
  __shared__ LDS_ALIGN T As[2][BT * LDT];           // rows of a (i)
  __shared__ LDS_ALIGN T Bs[2][BT * LDT];           // rows of b (j)

  const int64_t u = (int64_t)(blockIdx.x % 8) * per_xcd + blockIdx.x / 8;
  if (u >= units) return;
  const int64_t c = u / (tiles1 * tiles1);
  const int64_t tt = u - c * tiles1 * tiles1;
  const int64_t i0 = (tt / tiles1) * BT, j0 = (tt % tiles1) * BT;
  const T* a = ab + c * N * ld;
  const T* b = ab + ((int64_t)D + c) * N * ld;
  const int t = threadIdx.x, wave = t >> 6, l = t & 63, g = l >> 4;
  const int wi = wave >> 1, wj = wave & 1;

  // stage loads: vector v of thread t covers row (v*256 + t) / VPR of [a rows | b rows], column ((..) % VPR) * VE
  u32x4_t reg[LOADS];
  auto gload = [&](int64_t k0) {
#pragma unroll
    for (int v = 0; v < LOADS; v++) {
      const int e = v * 256 + t, r = e / VPR, col = (e % VPR) * VE;
      const bool isb = r >= BT;
      int64_t row = (isb ? j0 : i0) + (isb ? r - BT : r);
      if (row >= N) row = N - 1;
      reg[v] = *reinterpret_cast<const u32x4_t*>((isb ? b : a) + row * ld + k0 + col);
    }
  };
  auto lstore = [&](int buf) {
#pragma unroll
    for (int v = 0; v < LOADS; v++) {
      const int e = v * 256 + t, r = e / VPR, col = (e % VPR) * VE;
      T* dst = r >= BT ? Bs[buf] + (r - BT) * LDT : As[buf] + r * LDT;
      *reinterpret_cast<u32x4_t*>(dst + col) = reg[v];
    }
  };

  f4 acc[4][4];  // acc[jb][ib]: o^T block (j = 64*wj + 16*jb .., i = 64*wi + 16*ib ..)
  zero_acc(acc);
  gload(0);
  lstore(0);
  __syncthreads();
  for (int st = 0; st < nst; st++) {
    const int buf = st & 1;
    if (st + 1 < nst) gload((int64_t)(st + 1) * BK);
    const T* Ab = As[buf];
    const T* Bb = Bs[buf];
#pragma unroll
    for (int s = 0; s < STEPS; s++) {
      typename Mfma<T>::frag fa[4], fb[4];
#pragma unroll
      for (int ib = 0; ib < 4; ib++)
        fa[ib] = Mfma<T>::load(Ab + (64 * wi + 16 * ib + (l & 15)) * LDT + KG * g + KP * s);
#pragma unroll
      for (int jb = 0; jb < 4; jb++)
        fb[jb] = Mfma<T>::load(Bb + (64 * wj + 16 * jb + (l & 15)) * LDT + KG * g + KP * s);
#pragma unroll
      for (int jb = 0; jb < 4; jb++)
#pragma unroll
        for (int ib = 0; ib < 4; ib++) acc[jb][ib] = Mfma<T>::run(fb[jb], fa[ib], acc[jb][ib]);
    }
    if (st + 1 < nst) lstore(buf ^ 1);
    __syncthreads();
  }
  // acc[jb][ib][e] = o[i = i0 + 64 wi + 16 ib + (l & 15)][j = j0 + 64 wj + 16 jb + 4 g + e]
  T* oc = o + c * N * ld;
#pragma unroll
  for (int ib = 0; ib < 4; ib++) {
    const int64_t i = i0 + 64 * wi + 16 * ib + (l & 15);
    if (i >= N) continue;
#pragma unroll
    for (int jb = 0; jb < 4; jb++) {
      const int64_t j = j0 + 64 * wj + 16 * jb + 4 * g;
      if (j >= ld) continue;
      T* dst = oc + i * ld + j;
      if constexpr (sizeof(T) == 2) {
        *reinterpret_cast<half4*>(dst) =
            half4{(half_t)acc[jb][ib][0], (half_t)acc[jb][ib][1], (half_t)acc[jb][ib][2], (half_t)acc[jb][ib][3]};
      } else {
        *reinterpret_cast<f4*>(dst) = acc[jb][ib];
      }
    }
  }
}

// fp16 form, persistent and LDS-direct. One 512-thread workgroup per CU walks its tiles (256 x 256 of one channel) as
// one stream of K stages, so the next tile's first stages load while the current tile's last stages compute. A tile
// is 8 waves of 128 (j) x 64 (i) = 4 x 2 blocks of 32 x 32 on v_mfma_f32_32x32x16_f16 (128 accumulator registers per
// lane, 2 waves per SIMD). K stages of BK elements go from memory straight into LDS (buffer_load ... lds: no staging
// registers, no LDS store instructions), NS stages deep. A wave's load instruction fills 1 KB of LDS in lane order,
// so the LDS row layout is fixed; each lane picks its global 16-byte chunk so that LDS chunk p of row R holds the
// row's chunk p ^ swz(R), which makes the fragment reads (16 lanes on 16 rows at one logical chunk) hit distinct
// banks. The fragments of MFMA step g + 1 are read while step g computes (two register sets, across stage
// boundaries too) and the reads are interleaved with the MFMAs. The output tile leaves through a small LDS buffer so
// that each store instruction writes whole 128-byte row segments (scattered 8-byte stores took a third of the time).
// The lane-to-k assignment (lane half h takes k = 32 h + 8 s .. + 7 of a 64-element stage in step s) is the one the
// earlier register-staged kernel used, so the accumulation order, and the result, are unchanged.
// (ct_swz, in bzpf_layout.h: the swizzle of a row, checked on the host for bijectivity and bank conflicts)

template <int BK, int NS>
__global__ __launch_bounds__(512, 1) void trimul_contract_f16_k(const half_t* __restrict__ ab, half_t* __restrict__ o,
                                                                int64_t N, int64_t ld, int D, int64_t tiles1,
                                                                int64_t units, int64_t per_xcd, int wg_per_xcd,
                                                                int nst) {
  constexpr int BT = 256, NW = 8;
  constexpr int ROWB = BK * 2;               // bytes of a row per stage
  constexpr int CPR = ROWB / 16;             // 16-byte chunks per row
  constexpr int RPI = 1024 / ROWB;           // rows per load instruction
  constexpr int STAGE = 2 * BT * ROWB;       // a rows, then b rows
  constexpr int LPW = 2 * BT / RPI / NW;     // load instructions per wave per stage (first half a, second half b)
  constexpr int STEPS = BK / 16;
  // the stage slots, then one 4 KB output staging buffer per wave (160 KB)
  __shared__ __attribute__((aligned(1024))) char lds[NS * STAGE + NW * 4096];

  // this workgroup's tiles: u = first + wg_per_xcd * k, k < cnt, inside its XCD's contiguous range of units (the
  // XCD's CUs work on consecutive tiles, so one channel's a and b stay in its L2)
  const int xcd = blockIdx.x % 8;
  const int64_t first = (int64_t)xcd * per_xcd + blockIdx.x / 8;
  const int64_t end = min(units, (int64_t)(xcd + 1) * per_xcd);
  if (first >= end) return;
  const int cnt = (int)((end - first + wg_per_xcd - 1) / wg_per_xcd);
  const int total = cnt * nst;

  const int t = threadIdx.x, w = t >> 6, l = t & 63, r = l & 31, h = l >> 5;
  const int wj = w >> 2, wi = w & 3;  // wave tile: j = 128 wj .., i = 64 wi ..
  struct Tile { int64_t c, i0, j0; };
  auto tile = [&](int k) {
    const int64_t u = first + (int64_t)wg_per_xcd * k;
    const int64_t c = u / (tiles1 * tiles1);
    const int64_t tt = u - c * tiles1 * tiles1;
    return Tile{c, (tt / tiles1) * BT, (tt % tiles1) * BT};
  };

  constexpr int RSRC_CFG = 0x00020000;
  const int chan_bytes = (int)contract_extent(N, ld);
  // lane part of every load: row w * RPI + l / CPR of its 8-wave group, logical chunk (l % CPR) ^ swz(row)
  const int lrow = w * RPI + l / CPR;
  const int voff = (int)(((int64_t)lrow * ld + 8 * ((l % CPR) ^ ct_swz<BK>(lrow))) * 2);
  // The row part of the offset rides in the lane offset, which the buffer range check covers: rows past N read as
  // zeros (their outputs are not stored) and nothing is read past the end of a channel. The stage's k rides in the
  // scalar offset. Global stage gs = k * nst + stage; issues past the last one reload it (into a slot never read).
  auto issue = [&](int gs, int slot) {
    gs = min(gs, total - 1);
    const int k = gs / nst, stage = gs - k * nst;
    const Tile tl = tile(k);
    const __amdgpu_buffer_rsrc_t ars =
        __builtin_amdgcn_make_buffer_rsrc((void*)(ab + tl.c * N * ld), 0, chan_bytes, RSRC_CFG);
    const __amdgpu_buffer_rsrc_t brs =
        __builtin_amdgcn_make_buffer_rsrc((void*)(ab + ((int64_t)D + tl.c) * N * ld), 0, chan_bytes, RSRC_CFG);
    char* dst = lds + slot * STAGE + w * 1024;
#pragma unroll
    for (int v = 0; v < LPW; v++) {
      const bool isa = v < LPW / 2;
      const int64_t row0 = (isa ? tl.i0 : tl.j0) + (int64_t)(v % (LPW / 2)) * NW * RPI;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(isa ? ars : brs,
                                               (__attribute__((address_space(3))) void*)(dst + v * NW * 1024), 16,
                                               voff + (int)(row0 * ld * 2), stage * BK * 2, 0, 0);
    }
  };

  f16x acc[4][2];  // acc[jb][ib]: o^T block (j = 128 wj + 32 jb .., i = 64 wi + 32 ib ..)
  auto zero = [&]() {
#pragma unroll
    for (int jb = 0; jb < 4; jb++)
#pragma unroll
      for (int ib = 0; ib < 2; ib++)
#pragma unroll
        for (int e = 0; e < 16; e++) acc[jb][ib][e] = 0.0f;
  };
  // acc[jb][ib][4 q + e] = o[i = i0 + 64 wi + 32 ib + r][j = j0 + 128 wj + 32 jb + 8 q + 4 h + e]
  // Stores through a wave-private LDS buffer: each 32 (i) x 64 (j) piece of the wave's tile is written in the
  // accumulator layout (16-byte chunks XOR-swizzled by row) and read back as 16 bytes of one row per lane, so a
  // store instruction covers 8 rows x 128 contiguous bytes rather than 32 rows x 16 bytes.
  char* ob = lds + NS * STAGE + w * 4096;
  auto store = [&](int k) {
    const Tile tl = tile(k);
    half_t* oc = o + tl.c * N * ld;
#pragma unroll
    for (int ib = 0; ib < 2; ib++)
#pragma unroll
      for (int jp = 0; jp < 2; jp++) {
#pragma unroll
        for (int jj = 0; jj < 2; jj++)
#pragma unroll
          for (int q = 0; q < 4; q++) {
            const f16x& v = acc[2 * jp + jj][ib];
            *reinterpret_cast<half4*>(ob + r * 128 + (((4 * jj + q) ^ (r & 7)) * 16) + 8 * h) =
                half4{(half_t)v[4 * q], (half_t)v[4 * q + 1], (half_t)v[4 * q + 2], (half_t)v[4 * q + 3]};
          }
#pragma unroll
        for (int rr = 0; rr < 4; rr++) {
          const int R = (l >> 3) + 8 * rr;
          const u32x4_t val = *reinterpret_cast<const u32x4_t*>(ob + R * 128 + (((l & 7) ^ (R & 7)) * 16));
          const int64_t i = tl.i0 + 64 * wi + 32 * ib + R;
          const int64_t j = tl.j0 + 128 * wj + 64 * jp + 8 * (l & 7);
          if (i < N && j < ld) *reinterpret_cast<u32x4_t*>(oc + i * ld + j) = val;
        }
      }
  };
  zero();
  const int sw = ct_swz<BK>(r);  // rows read by this lane: (block base, a multiple of 32) + r
  // fragment sets: the reads of MFMA step g + 1 are issued before the MFMAs of step g (two register sets), across
  // stage boundaries too, so each wave's own MFMAs cover its LDS latency and the barrier
  half8 fa[2][4], fb[2][2];
  auto read = [&](int set, int slot, int s) {
    const char* base = lds + slot * STAGE;
    const int chunk = (STEPS * h + s) ^ sw;
#pragma unroll
    for (int jb = 0; jb < 4; jb++)
      fa[set][jb] = *reinterpret_cast<const half8*>(base + (BT + 128 * wj + 32 * jb + r) * ROWB + 16 * chunk);
#pragma unroll
    for (int ib = 0; ib < 2; ib++)
      fb[set][ib] = *reinterpret_cast<const half8*>(base + (64 * wi + 32 * ib + r) * ROWB + 16 * chunk);
  };
  auto mfma = [&](int set) {
#pragma unroll
    for (int jb = 0; jb < 4; jb++)
#pragma unroll
      for (int ib = 0; ib < 2; ib++)
        acc[jb][ib] = __builtin_amdgcn_mfma_f32_32x32x16_f16(fa[set][jb], fb[set][ib], acc[jb][ib], 0, 0, 0);
  };
  // stages gs + 1 .. gs + NS - 1 are in flight while stage gs computes, so every wave always has (NS - 2) * LPW
  // loads younger than the stage it waits for
  constexpr int YOUNGER = (NS - 2) * LPW;
  constexpr int WAIT = (YOUNGER & 15) | ((YOUNGER >> 4) << 14) | (0x7 << 4) | (0xF << 8);  // vmcnt only
#pragma unroll
  for (int p = 0; p < NS - 1; p++) issue(p, p);
  __builtin_amdgcn_s_waitcnt(WAIT);  // stage 0 has landed (this wave's part)
  __builtin_amdgcn_s_barrier();      // (everyone's)
  __builtin_amdgcn_sched_barrier(0);
  issue(NS - 1, NS - 1);
  read(0, 0, 0);
  int stage = 0, k = 0;
  for (int gs = 0; gs < total; gs++) {
    const int slot = gs % NS;
#pragma unroll
    for (int s = 0; s < STEPS; s++) {
      const int cur = s & 1;  // STEPS is even: step 0 of every stage uses set 0
      if (s + 1 < STEPS) {
        read(cur ^ 1, slot, s + 1);
      } else if (gs + 1 < total) {
        // every read of this slot by this wave is done (the last set is in registers) and stage gs + 1 has landed;
        // after the barrier the slot takes stage gs + NS
        __builtin_amdgcn_s_waitcnt(WAIT & ~(0xF << 8));  // vmcnt as above, lgkmcnt(0)
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_sched_barrier(0);
        issue(gs + NS, slot);
        read(cur ^ 1, (gs + 1) % NS, 0);
      }
      mfma(cur);
      // interleave: the next set's LDS reads between this set's MFMAs
#pragma unroll
      for (int q = 0; q < 6; q++) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
      }
      __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
    }
    if (++stage == nst) {  // tile k done: its stores drain while the next tile computes
      store(k);
      zero();
      stage = 0;
      k++;
    }
  }
  __builtin_amdgcn_s_waitcnt(0);  // no LDS write of a trailing (unused) stage load outlives the workgroup
}

// kl: the k range contracted (a multiple of the stage width, <= ld); columns past it are zero in a and b.
template <typename T>
static hipError_t contract_t(const void* ab, void* o, int64_t N, int64_t ld, int64_t kl, int D, hipStream_t st) {
  const int BT = sizeof(T) == 2 ? 256 : 128;
  const int64_t tiles1 = (N + BT - 1) / BT;
  const int64_t units = (int64_t)D * tiles1 * tiles1;
  const int64_t per_xcd = (units + 7) / 8;
  const dim3 grid((unsigned)(per_xcd * 8));
  if constexpr (sizeof(T) == 2) {
    static int cache[kMaxDevices] = {};
    const int resident = resident_grid(trimul_contract_f16_k<64, 2>, 512, cache);
    if (resident < 8) return hipErrorInvalidConfiguration;
    const int wpx = (int)(resident / 8 < per_xcd ? resident / 8 : per_xcd);
    trimul_contract_f16_k<64, 2><<<dim3(8 * wpx), 512, 0, st>>>(static_cast<const half_t*>(ab), static_cast<half_t*>(o),
                                                               N, ld, D, tiles1, units, per_xcd, wpx, (int)(kl / 64));
  } else {
    trimul_contract_kernel<T><<<grid, 256, 0, st>>>(static_cast<const T*>(ab), static_cast<T*>(o), N, ld, D, tiles1,
                                                    units, per_xcd, (int)(kl / 32));
  }
  return hipGetLastError();
}

hipError_t launch_trimul_contract(const void* ab, void* o, int dt, int64_t N, int64_t ld, int64_t k_len, int D,
                                  hipStream_t st) {
  if (dt == DT_F16 && !contract_shape_ok(N, ld)) return hipErrorInvalidValue;  // 32-bit buffer offsets per channel
  // contract over k < k_len rounded up to 64 (a whole number of stages of either kernel); 0 or >= N: every k
  const int64_t kl = k_len <= 0 || k_len >= N ? ld : (k_len + 63) / 64 * 64;
  return dt == DT_F16 ? contract_t<half_t>(ab, o, N, ld, kl, D, st) : contract_t<float>(ab, o, N, ld, kl, D, st);
}

}  // namespace bzpf
