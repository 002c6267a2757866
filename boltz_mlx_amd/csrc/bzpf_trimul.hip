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
                                                                 int64_t units, int64_t per_xcd) {
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
  const int nst = (int)(ld / BK);
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

// fp16 form: 256 x 256 tiles on v_mfma_f32_32x32x16_f16, 16 waves of 64 (j) x 64 (i) = 2 x 2 blocks of 32 x 32
// (64 accumulator registers per lane, 4 waves per SIMD). The 128 x 128 tile of the fp32 form moves 32 KB from L2 per
// 2.1 MFLOP; this tile halves that (64 KB per 8.4 MFLOP per 64-element K stage). K stages (64 elements) are
// double-buffered in LDS (147 KB, one workgroup per CU); two register sets carry the next two stages, so each load
// has two stages of compute to land (one stage, about 1 us, is shorter than the loaded L2/HBM latency); four waves
// per SIMD (rather than two with 128 x 64 wave tiles) keep the matrix cores busier through each stage's barrier and
// LDS waits.
// Operand layouts (A = rows of b, B = rows of a, both K-contiguous): lane l holds row l % 32 and 8 consecutive k;
// in MFMA step s of a stage, lane half h = l / 32 takes k = 32 h + 8 s .. + 7, so over the 4 steps a lane reads 64
// contiguous bytes of its row (a permutation of the k sum shared by A and B). The accumulator lane holds
// o^T[j = 8 q + 4 h + e][i = l % 32] in element 4 q + e: 4 runs of 4 consecutive j of one i.
constexpr int CT_BT = 256, CT_WAVES = 16;

__global__ __launch_bounds__(64 * CT_WAVES, 1) void trimul_contract_f16_k(const half_t* __restrict__ ab,
                                                                          half_t* __restrict__ o, int64_t N,
                                                                          int64_t ld, int D, int64_t tiles1,
                                                                          int64_t units, int64_t per_xcd) {
  constexpr int BT = CT_BT, BK = 64, NT = 64 * CT_WAVES;
  constexpr int LDT = BK + 8;              // LDS row pitch (halves): 36 dwords, conflict-free 16-byte row reads
  constexpr int VPR = BK / 8;              // 16-byte vectors per row per stage
  constexpr int LOADS = 2 * BT * VPR / NT;  // 8
  __shared__ LDS_ALIGN half_t As[2][BT * LDT];  // rows of a (i)
  __shared__ LDS_ALIGN half_t Bs[2][BT * LDT];  // rows of b (j)

  const int64_t u = (int64_t)(blockIdx.x % 8) * per_xcd + blockIdx.x / 8;
  if (u >= units) return;
  const int64_t c = u / (tiles1 * tiles1);
  const int64_t tt = u - c * tiles1 * tiles1;
  const int64_t i0 = (tt / tiles1) * BT, j0 = (tt % tiles1) * BT;
  const half_t* a = ab + c * N * ld;
  const half_t* b = ab + ((int64_t)D + c) * N * ld;
  const int t = threadIdx.x, wave = t >> 6, l = t & 63, r = l & 31, h = l >> 5;
  const int wj = wave >> 2, wi = wave & 3;  // wave tile: j = 64 wj .., i = 64 wi ..

  // Staging: thread t moves 16-byte vector (t / 8, 8 (t % 8)) of each 128-row quarter: quarters 0, 1 of a (rows
  // i0 ..), 2, 3 of b (rows j0 ..). Loads go through buffer resources: the lane offset is fixed, the quarter's rows
  // and the stage's k ride in the scalar offset, and rows past N read as zeros (range check; those outputs are not
  // stored).
  constexpr int RSRC_CFG = 0x00020000;  // raw buffer, 32-bit data format
  const __amdgpu_buffer_rsrc_t ars = __builtin_amdgcn_make_buffer_rsrc((void*)a, 0, (int)(N * ld * 2), RSRC_CFG);
  const __amdgpu_buffer_rsrc_t brs = __builtin_amdgcn_make_buffer_rsrc((void*)b, 0, (int)(N * ld * 2), RSRC_CFG);
  const int voff = (int)(((t >> 3) * ld + (t & 7) * 8) * 2);
  const int loff = (t >> 3) * LDT + (t & 7) * 8;  // LDS element offset inside a quarter
  // two register sets: stage s + 2 is loaded while stage s computes, so each load has two stages of time to land
  u32x4_t reg0[LOADS], reg1[LOADS];
  auto gload = [&](u32x4_t (&reg)[LOADS], int stage) {
#pragma unroll
    for (int v = 0; v < LOADS; v++) {
      const int so = (int)((((v < 2 ? i0 : j0) + 128 * (v & 1)) * ld + (int64_t)stage * BK) * 2);
      reg[v] = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(v < 2 ? ars : brs, voff, so, 0));
    }
  };
  auto lstore = [&](const u32x4_t (&reg)[LOADS], int buf) {
#pragma unroll
    for (int v = 0; v < LOADS; v++)
      *reinterpret_cast<u32x4_t*>((v < 2 ? As[buf] : Bs[buf]) + 128 * (v & 1) * LDT + loff) = reg[v];
  };

  f16x acc[2][2];  // acc[jb][ib]: o^T block (j = 64 wj + 32 jb .., i = 64 wi + 32 ib ..)
#pragma unroll
  for (int jb = 0; jb < 2; jb++)
#pragma unroll
    for (int ib = 0; ib < 2; ib++)
#pragma unroll
      for (int e = 0; e < 16; e++) acc[jb][ib][e] = 0.0f;
  auto compute = [&](int buf) {
    const half_t* Ab = As[buf] + (64 * wi + r) * LDT + 32 * h;
    const half_t* Bb = Bs[buf] + (64 * wj + r) * LDT + 32 * h;
#pragma unroll
    for (int s = 0; s < 4; s++) {
      half8 fa[2], fb[2];
#pragma unroll
      for (int q = 0; q < 2; q++) fa[q] = *reinterpret_cast<const half8*>(Ab + 32 * q * LDT + 8 * s);
#pragma unroll
      for (int q = 0; q < 2; q++) fb[q] = *reinterpret_cast<const half8*>(Bb + 32 * q * LDT + 8 * s);
#pragma unroll
      for (int jb = 0; jb < 2; jb++)
#pragma unroll
        for (int ib = 0; ib < 2; ib++)
          acc[jb][ib] = __builtin_amdgcn_mfma_f32_32x32x16_f16(fb[jb], fa[ib], acc[jb][ib], 0, 0, 0);
    }
  };
  const int nst = (int)(ld / BK);
  // Stages pair up (buffer 0, buffer 1) per trip; an odd stage count starts with a zero stage in buffer 0 (adds
  // nothing), so the trip body has no branch and the wait counter sees one load order. Loads past the last stage
  // reload it into registers that are never stored.
  const int s0 = -(nst & 1);
  gload(reg0, 0);
#pragma unroll
  for (int v = 0; v < LOADS; v++) reg0[v] = s0 ? u32x4_t{0u, 0u, 0u, 0u} : reg0[v];
  lstore(reg0, 0);
  __syncthreads();
  // issue order pinned (reg0 before reg1, as in the loop): the wait counter then needs only the older set
  gload(reg0, s0 + 1);
  __builtin_amdgcn_sched_barrier(0);
  gload(reg1, min(s0 + 2, nst - 1));
  __builtin_amdgcn_sched_barrier(0);
  for (int st = s0; st < nst; st += 2) {
    compute(0);       // stage st
    lstore(reg0, 1);  // stage st + 1
    __syncthreads();
    gload(reg0, min(st + 3, nst - 1));
    __builtin_amdgcn_sched_barrier(0);
    compute(1);       // stage st + 1
    lstore(reg1, 0);  // stage st + 2
    __syncthreads();
    gload(reg1, min(st + 4, nst - 1));
    __builtin_amdgcn_sched_barrier(0);
  }
  half_t* oc = o + c * N * ld;
#pragma unroll
  for (int ib = 0; ib < 2; ib++) {
    const int64_t i = i0 + 64 * wi + 32 * ib + r;
    if (i >= N) continue;
#pragma unroll
    for (int jb = 0; jb < 2; jb++)
#pragma unroll
      for (int q = 0; q < 4; q++) {
        const int64_t j = j0 + 64 * wj + 32 * jb + 8 * q + 4 * h;
        if (j >= ld) continue;
        const f16x& v = acc[jb][ib];
        *reinterpret_cast<half4*>(oc + i * ld + j) =
            half4{(half_t)v[4 * q], (half_t)v[4 * q + 1], (half_t)v[4 * q + 2], (half_t)v[4 * q + 3]};
      }
  }
}

template <typename T>
static hipError_t contract_t(const void* ab, void* o, int64_t N, int64_t ld, int D, hipStream_t st) {
  const int BT = sizeof(T) == 2 ? CT_BT : 128;
  const int64_t tiles1 = (N + BT - 1) / BT;
  const int64_t units = (int64_t)D * tiles1 * tiles1;
  const int64_t per_xcd = (units + 7) / 8;
  const dim3 grid((unsigned)(per_xcd * 8));
  if constexpr (sizeof(T) == 2)
    trimul_contract_f16_k<<<grid, 64 * CT_WAVES, 0, st>>>(static_cast<const half_t*>(ab), static_cast<half_t*>(o), N,
                                                          ld, D, tiles1, units, per_xcd);
  else
    trimul_contract_kernel<T><<<grid, 256, 0, st>>>(static_cast<const T*>(ab), static_cast<T*>(o), N, ld, D, tiles1,
                                                    units, per_xcd);
  return hipGetLastError();
}

hipError_t launch_trimul_contract(const void* ab, void* o, int dt, int64_t N, int64_t ld, int D, hipStream_t st) {
  if (dt == DT_F16 && 2 * N * ld >= (1LL << 31)) return hipErrorInvalidValue;  // 32-bit buffer offsets per channel
  return dt == DT_F16 ? contract_t<half_t>(ab, o, N, ld, D, st) : contract_t<float>(ab, o, N, ld, D, st);
}

}  // namespace bzpf
