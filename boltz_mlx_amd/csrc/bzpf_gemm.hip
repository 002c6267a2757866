// Row GEMM (fp16 or fp32 operands) with fused epilogues for the linear layers of the s track and the diffusion transformer:
//   y[r][m] = x[r] . W[m] + bias[m]                     (epi 0: stored as fp16 or fp32)
//   y[r][m] += x[r] . W[m] + bias[m]                    (epi 1: fp32 y)
//   y[r][m] += sigmoid(gate[r % gate_rows][m]) * (..)   (epi 2: fp32 y, the diffusion transformer's gated residuals)
//   y[r][m] = res[r][m] + x[r] . W[m] + bias[m]         (epi 3: fp32 y, res passed as `gate` with pitch ld_gate: an
//                                                        update written out of place, same sums as a copy + epi 1)
// with x [R][K] and W [M][K] both K-contiguous (nn.Linear), K a multiple of 128 bytes (64 fp16 / 32 fp32 elements).
// Reference behaviour: the nn.Linear / lin16 calls these replace (boltz_mlx/kernels.py:1360-1370;
// boltz_mlx/modules/transformersv2.py:199-264).
//
// A 256-thread workgroup owns a BM x BR tile of y^T (BM, BR = 64 or 128; gemm_tile_choice picks), 4 waves of
// BM / 2 x BR / 2 on v_mfma_f32_32x32x16_f16. The tile is computed transposed (y^T = W x^T: A = rows of W, B = rows
// of x), so an accumulator lane holds 4 runs of 4 consecutive output columns of one row and stores 8- or 16-byte
// vectors. K stages of 64 are double-buffered in LDS (36-72 KB) and two register sets carry the next two stages.
// gemm_lds_k is the same computation with the stages loaded straight into LDS, three deep (the default below the
// large-grid case).
// Rows of x past R and rows of W past M read as zeros through the buffer range check; their outputs are not stored.
#include "bzpf_common.h"
#include "bzpf_kernels.h"

namespace bzpf {

namespace {

template <int BM, int BR, typename TX, typename TY>
__global__ __launch_bounds__(256, 2) void gemm_nt_k(const TX* __restrict__ x, const TX* __restrict__ w,
                                                    const float* __restrict__ bias, TY* __restrict__ y, int64_t R,
                                                    int K, int M, int epi, const float* __restrict__ gate,
                                                    int64_t ld_gate, int64_t gate_rows) {
  static_assert((BM == 64 || BM == 128) && (BR == 64 || BR == 128), "64- or 128-row tiles");
  constexpr int ES = sizeof(TX), VE = 16 / ES;  // element size, elements per 16-byte vector
  constexpr int BK = 128 / ES, LDT = BK + VE;   // a stage is 128 bytes of each row (64 fp16 or 32 fp32 elements)
  constexpr int LA = BM / 32, LB = BR / 32;  // 16-byte vectors per thread per stage: rows of W, rows of x
  constexpr int MB = BM / 64, RB = BR / 64;  // 32 x 32 MFMA blocks per wave along m and r
  __shared__ LDS_ALIGN TX As[2][BM * LDT];  // rows of W (m)
  __shared__ LDS_ALIGN TX Bs[2][BR * LDT];  // rows of x (r)
  const int64_t r0 = (int64_t)blockIdx.x * BR;
  const int m0 = blockIdx.y * BM;
  const int t = threadIdx.x, wave = t >> 6, l = t & 63, rr = l & 31, hh = l >> 5;
  const int wm = wave >> 1, wr = wave & 1;  // wave tile: m = BM / 2 wm .., r = BR / 2 wr ..

  constexpr int RSRC_CFG = 0x00020000;
  const int64_t xrows = R - r0 < BR ? R - r0 : BR;
  const int wrows = M - m0 < BM ? M - m0 : BM;
  const __amdgpu_buffer_rsrc_t xrs =
      __builtin_amdgcn_make_buffer_rsrc((void*)(x + r0 * K), 0, (int)(xrows * K * ES), RSRC_CFG);
  const __amdgpu_buffer_rsrc_t wrs =
      __builtin_amdgcn_make_buffer_rsrc((void*)(w + (int64_t)m0 * K), 0, (int)((int64_t)wrows * K * ES), RSRC_CFG);
  // staging: vector v of thread t is row 32 v + t / 8 of its operand's tile, 16 bytes at k VE (t % 8) of the stage
  const int lrow = t >> 3, lcol = (t & 7) * VE;
  u32x4_t ra0[LA], rb0[LB], ra1[LA], rb1[LB];
  auto gload = [&](u32x4_t (&ra)[LA], u32x4_t (&rb)[LB], int stage) {
#pragma unroll
    for (int v = 0; v < LA; v++) {
      const int off = (int)(((int64_t)(32 * v + lrow) * K + stage * BK + lcol) * ES);
      ra[v] = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(wrs, off, 0, 0));
    }
#pragma unroll
    for (int v = 0; v < LB; v++) {
      const int off = (int)(((int64_t)(32 * v + lrow) * K + stage * BK + lcol) * ES);
      rb[v] = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(xrs, off, 0, 0));
    }
  };
  auto lstore = [&](const u32x4_t (&ra)[LA], const u32x4_t (&rb)[LB], int buf) {
#pragma unroll
    for (int v = 0; v < LA; v++) *reinterpret_cast<u32x4_t*>(As[buf] + (32 * v + lrow) * LDT + lcol) = ra[v];
#pragma unroll
    for (int v = 0; v < LB; v++) *reinterpret_cast<u32x4_t*>(Bs[buf] + (32 * v + lrow) * LDT + lcol) = rb[v];
  };
  f16x acc[MB][RB];  // acc[mb][rb]: y^T block (m = BM / 2 wm + 32 mb .., r = BR / 2 wr + 32 rb ..)
#pragma unroll
  for (int mb = 0; mb < MB; mb++)
#pragma unroll
    for (int rb = 0; rb < RB; rb++)
#pragma unroll
      for (int e = 0; e < 16; e++) acc[mb][rb][e] = 0.0f;
  // Lane half hh takes the contiguous half k = BK / 2 hh .. of each stage for both operands (a permutation of the
  // k sum): fp16, MFMA step s takes k = 32 hh + 8 s .. + 7 (v_mfma_f32_32x32x16_f16); fp32, step 4 s + e takes
  // k = 16 hh + 4 s + e (v_mfma_f32_32x32x2f32, one element per lane), read as one 16-byte vector per s.
  auto compute = [&](int buf) {
    const TX* Ab = As[buf] + (BM / 2 * wm + rr) * LDT + BK / 2 * hh;
    const TX* Bb = Bs[buf] + (BR / 2 * wr + rr) * LDT + BK / 2 * hh;
#pragma unroll
    for (int s = 0; s < 4; s++) {
      if constexpr (ES == 2) {
        half8 fa[MB], fb[RB];
#pragma unroll
        for (int q = 0; q < MB; q++) fa[q] = *reinterpret_cast<const half8*>(Ab + 32 * q * LDT + 8 * s);
#pragma unroll
        for (int q = 0; q < RB; q++) fb[q] = *reinterpret_cast<const half8*>(Bb + 32 * q * LDT + 8 * s);
#pragma unroll
        for (int mb = 0; mb < MB; mb++)
#pragma unroll
          for (int rb = 0; rb < RB; rb++)
            acc[mb][rb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(fa[mb], fb[rb], acc[mb][rb], 0, 0, 0);
      } else {
        f4 fa[MB], fb[RB];
#pragma unroll
        for (int q = 0; q < MB; q++) fa[q] = *reinterpret_cast<const f4*>(Ab + 32 * q * LDT + 4 * s);
#pragma unroll
        for (int q = 0; q < RB; q++) fb[q] = *reinterpret_cast<const f4*>(Bb + 32 * q * LDT + 4 * s);
#pragma unroll
        for (int e = 0; e < 4; e++)
#pragma unroll
          for (int mb = 0; mb < MB; mb++)
#pragma unroll
            for (int rb = 0; rb < RB; rb++)
              acc[mb][rb] = __builtin_amdgcn_mfma_f32_32x32x2f32(fa[mb][e], fb[rb][e], acc[mb][rb], 0, 0, 0);
      }
    }
  };
  const int nst = K / BK;
  // stages pair up (buffer 0, buffer 1); an odd count starts with a zero stage; loads past the last stage reload it
  const int s0 = -(nst & 1);
  gload(ra0, rb0, 0);
#pragma unroll
  for (int v = 0; v < LA; v++) ra0[v] = s0 ? u32x4_t{0u, 0u, 0u, 0u} : ra0[v];
#pragma unroll
  for (int v = 0; v < LB; v++) rb0[v] = s0 ? u32x4_t{0u, 0u, 0u, 0u} : rb0[v];
  lstore(ra0, rb0, 0);
  __syncthreads();
  gload(ra0, rb0, s0 + 1);
  __builtin_amdgcn_sched_barrier(0);
  gload(ra1, rb1, min(s0 + 2, nst - 1));
  __builtin_amdgcn_sched_barrier(0);
  for (int st = s0; st < nst; st += 2) {
    compute(0);
    lstore(ra0, rb0, 1);
    __syncthreads();
    gload(ra0, rb0, min(st + 3, nst - 1));
    __builtin_amdgcn_sched_barrier(0);
    compute(1);
    lstore(ra1, rb1, 0);
    __syncthreads();
    gload(ra1, rb1, min(st + 4, nst - 1));
    __builtin_amdgcn_sched_barrier(0);
  }
  // epilogue: lane (rr, hh) of block (mb, rb) holds y[r][m .. m + 3] for r = BR / 2 wr + 32 rb + rr and
  // m = BM / 2 wm + 32 mb + 8 q + 4 hh, q < 4
#pragma unroll
  for (int rb = 0; rb < RB; rb++) {
    const int64_t r = r0 + BR / 2 * wr + 32 * rb + rr;
    if (r >= R) continue;
#pragma unroll
    for (int mb = 0; mb < MB; mb++)
#pragma unroll
      for (int q = 0; q < 4; q++) {
        const int m = m0 + BM / 2 * wm + 32 * mb + 8 * q + 4 * hh;
        if (m >= M) continue;  // M % 4 == 0: a run of 4 is in or out whole
        f4 v4 = f4{acc[mb][rb][4 * q], acc[mb][rb][4 * q + 1], acc[mb][rb][4 * q + 2], acc[mb][rb][4 * q + 3]};
        if (bias != nullptr) v4 += *reinterpret_cast<const f4*>(bias + m);
        if (epi == 2) {
          const f4 gv = *reinterpret_cast<const f4*>(gate + (r % gate_rows) * ld_gate + m);
          v4 = f4{v4[0] * sigmoidf_(gv[0]), v4[1] * sigmoidf_(gv[1]), v4[2] * sigmoidf_(gv[2]),
                  v4[3] * sigmoidf_(gv[3])};
        }
        TY* yp = y + r * M + m;
        if constexpr (sizeof(TY) == 4) {
          if (epi == 3)
            v4 += *reinterpret_cast<const f4*>(gate + r * ld_gate + m);
          else if (epi >= 1)
            v4 += *reinterpret_cast<const f4*>(yp);
          *reinterpret_cast<f4*>(yp) = v4;
        } else {
          *reinterpret_cast<half4*>(yp) = half4{(half_t)v4[0], (half_t)v4[1], (half_t)v4[2], (half_t)v4[3]};
        }
      }
  }
}

// fp16 operands with the K stages loaded straight into LDS (buffer_load ... lds), NS stages deep: the same tiles,
// waves and lane-to-k assignment as gemm_nt_k (so the same sums in the same order), but NS - 1 stages in flight
// without staging registers. A wave's load instruction fills 1 KB of LDS in lane order (8 rows of 128 bytes); each
// lane picks the global 16-byte chunk that makes LDS chunk p of row R hold the row's chunk p ^ gl_swz(R), so the
// fragment reads (16 lanes on 16 consecutive rows at one logical chunk) hit distinct banks.
__device__ __forceinline__ int gl_swz(int row) { return (row & 7) ^ ((row >> 3) & 1); }

// SW = 2 or 3: the gated-product epilogue of gemm_swiglu_f16_k on the same tiles (BM = 64 SW, so each wave's BM / 2
// W rows are one group [W_0; W_1 (; W_2)] of 32 output columns); y is then the fp16 u [R][M / SW].
template <int BM, int BR, int NS, typename TY, int SW = 0>
__global__ __launch_bounds__(256, BM * BR > 128 * 64 ? 1 : 2) void gemm_lds_k(const half_t* __restrict__ x, const half_t* __restrict__ w,
                                                     const float* __restrict__ bias, TY* __restrict__ y, int64_t R,
                                                     int K, int M, int epi, const float* __restrict__ gate,
                                                     int64_t ld_gate, int64_t gate_rows, int nr, int nm, int per_xcd,
                                                     int mfast) {
  static_assert((BM == 64 || BM == 128 || BM == 192) && (BR == 64 || BR == 128) && NS >= 2, "tile / stages");
  static_assert(SW == 0 || (BM == 64 * SW && sizeof(TY) == 2), "gated product: one 32-column group per wave");
  constexpr int BK = 64, ROWB = 128, ROWS = BM + BR, STAGE = ROWS * ROWB;
  constexpr int LPW = ROWS / 32;             // load instructions per wave per stage (8 rows each, 4 waves)
  constexpr int MB = BM / 64, RB = BR / 64;  // 32 x 32 MFMA blocks per wave along m and r
  __shared__ __attribute__((aligned(1024))) char lds[NS * STAGE];
  // The nr x nm tiles are dealt to the 8 XCDs in contiguous ranges (the dispatcher sends workgroup b to XCD b % 8),
  // enumerated with the W tile fastest (mfast: an XCD's range holds a few x row tiles against all of W) or the x
  // tile fastest (a slice of W against all of x); the launcher picks the order whose per-XCD operand bytes are
  // fewer, so that they stay in the XCD's L2.
  const int u = (int)(blockIdx.x % 8) * per_xcd + (int)(blockIdx.x / 8);
  if (u >= nr * nm) return;  // whole workgroup
  const int rt = mfast ? u / nm : u % nr, mt = mfast ? u % nm : u / nr;
  const int64_t r0 = (int64_t)rt * BR;
  const int m0 = mt * BM;
  const int t = threadIdx.x, l = t & 63, rr = l & 31, hh = l >> 5;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const int wm = wave >> 1, wr = wave & 1;  // wave tile: m = BM / 2 wm .., r = BR / 2 wr ..

  constexpr int RSRC_CFG = 0x00020000;
  const int64_t xrows = R - r0 < BR ? R - r0 : BR;
  const int wrows = M - m0 < BM ? M - m0 : BM;
  const __amdgpu_buffer_rsrc_t xrs =
      __builtin_amdgcn_make_buffer_rsrc((void*)(x + r0 * K), 0, (int)(xrows * K * 2), RSRC_CFG);
  const __amdgpu_buffer_rsrc_t wrs =
      __builtin_amdgcn_make_buffer_rsrc((void*)(w + (int64_t)m0 * K), 0, (int)((int64_t)wrows * K * 2), RSRC_CFG);
  // instruction v of this wave fills stage rows 8 (4 v + wave) .. + 7: W rows [0, BM), then x rows [BM, ROWS)
  const int nst = K / BK;
  auto issue = [&](int st, int slot) {
    st = min(st, nst - 1);  // issues past the last stage reload it into a slot that is never read
#pragma unroll
    for (int v = 0; v < LPW; v++) {
      const int row = 8 * (4 * v + wave) + (l >> 3);
      const bool isw = 8 * (4 * v + wave) < BM;  // wave-uniform
      const int rloc = isw ? row : row - BM;
      const int voff = (rloc * K + 8 * ((l & 7) ^ gl_swz(row))) * 2;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          isw ? wrs : xrs, (__attribute__((address_space(3))) void*)(lds + slot * STAGE + (4 * v + wave) * 1024), 16,
          voff, st * BK * 2, 0, 0);
    }
  };
  f16x acc[MB][RB];
#pragma unroll
  for (int mb = 0; mb < MB; mb++)
#pragma unroll
    for (int rb = 0; rb < RB; rb++)
#pragma unroll
      for (int e = 0; e < 16; e++) acc[mb][rb][e] = 0.0f;
  // lane half hh takes k = 32 hh + 8 s .. + 7 of the stage in MFMA step s (gemm_nt_k's order)
  half8 fa[2][MB], fb[2][RB];
  auto read = [&](int set, int slot, int s) {
    const char* base = lds + slot * STAGE;
#pragma unroll
    for (int mb = 0; mb < MB; mb++) {
      const int row = BM / 2 * wm + 32 * mb + rr;
      fa[set][mb] = *reinterpret_cast<const half8*>(base + row * ROWB + 16 * ((4 * hh + s) ^ gl_swz(row)));
    }
#pragma unroll
    for (int rb = 0; rb < RB; rb++) {
      const int row = BM + BR / 2 * wr + 32 * rb + rr;
      fb[set][rb] = *reinterpret_cast<const half8*>(base + row * ROWB + 16 * ((4 * hh + s) ^ gl_swz(row)));
    }
  };
  // The epilogue's fp32 inputs (the y it accumulates into and the gate) are loaded before the K loop, so their
  // latency overlaps the loop instead of following the last stage (for the 768-wide gated outputs the epilogue is a
  // 12 MB read-modify-write). They are issued ahead of the stage loads: the loop's vmcnt waits count loads in issue
  // order, so these complete by the first stage's wait and never hold back a later one.
  // (tiles of up to two MFMA blocks per wave: larger ones would hold too many registers through the loop)
  constexpr bool PRE = sizeof(TY) == 4 && MB * RB <= 2;
  f4 ypre[RB][MB][4], gpre[RB][MB][4];
  if constexpr (PRE) {
#pragma unroll
    for (int rb = 0; rb < RB; rb++) {
      const int64_t r = r0 + BR / 2 * wr + 32 * rb + rr;
      const bool rin = r < R;
      const float* grow = epi == 2 && rin ? gate + (r % gate_rows) * ld_gate : nullptr;
#pragma unroll
      for (int mb = 0; mb < MB; mb++)
#pragma unroll
        for (int q = 0; q < 4; q++) {
          const int m = m0 + BM / 2 * wm + 32 * mb + 8 * q + 4 * hh;
          const bool in = rin && m < M;
          const float* src = epi == 3 ? gate + r * ld_gate + m : y + r * M + m;  // the residual's source
          ypre[rb][mb][q] = in && epi >= 1 ? *reinterpret_cast<const f4*>(src) : f4{0.f, 0.f, 0.f, 0.f};
          gpre[rb][mb][q] = in && grow != nullptr ? *reinterpret_cast<const f4*>(grow + m) : f4{0.f, 0.f, 0.f, 0.f};
        }
    }
  }
  __builtin_amdgcn_sched_barrier(0);
  constexpr int YOUNGER = (NS - 2) * LPW;  // loads of later stages in flight when a stage is waited for
  constexpr int WAIT = (YOUNGER & 15) | ((YOUNGER >> 4) << 14) | (0x7 << 4) | (0xF << 8);  // vmcnt only
#pragma unroll
  for (int p = 0; p < NS - 1; p++) issue(p, p);
  __builtin_amdgcn_s_waitcnt(WAIT);
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_sched_barrier(0);
  issue(NS - 1, NS - 1);
  read(0, 0, 0);
  for (int st = 0; st < nst; st++) {
    const int slot = st % NS;
#pragma unroll
    for (int s = 0; s < 4; s++) {
      const int cur = s & 1;
      if (s < 3) {
        read(cur ^ 1, slot, s + 1);
      } else if (st + 1 < nst) {
        // this wave's reads of the slot are done and stage st + 1 has landed; after the barrier the slot takes
        // stage st + NS
        __builtin_amdgcn_s_waitcnt(WAIT & ~(0xF << 8));  // vmcnt as above, lgkmcnt(0)
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_sched_barrier(0);
        issue(st + NS, slot);
        read(cur ^ 1, (st + 1) % NS, 0);
      }
#pragma unroll
      for (int mb = 0; mb < MB; mb++)
#pragma unroll
        for (int rb = 0; rb < RB; rb++)
          acc[mb][rb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(fa[cur][mb], fb[cur][rb], acc[mb][rb], 0, 0, 0);
    }
  }
  __builtin_amdgcn_s_waitcnt(0);  // the reloads past the last stage land before the workgroup's LDS is released
  if constexpr (SW != 0) {
    // gated product: the wave's blocks mb hold product mb of columns 32 grp .. + 31, grp = (m0 + BM / 2 wm) / 32 SW;
    // lane (rr, hh) holds columns 32 grp + 8 q + 4 hh .. + 3 in elements 4 q .. 4 q + 3 (gemm_swiglu_f16_k's order)
    const int H = M / SW, grp = (m0 + BM / 2 * wm) / (32 * SW);
    if (32 * grp >= H) return;
#pragma unroll
    for (int rb = 0; rb < RB; rb++) {
      const int64_t r = r0 + BR / 2 * wr + 32 * rb + rr;
      if (r >= R) continue;
#pragma unroll
      for (int q = 0; q < 4; q++) {
        half4 o;
#pragma unroll
        for (int e = 0; e < 4; e++) {
          float val = siluf_(acc[0][rb][4 * q + e]) * acc[1][rb][4 * q + e];
          if constexpr (SW == 3) val *= acc[2][rb][4 * q + e];
          o[e] = (half_t)val;
        }
        *reinterpret_cast<half4*>(y + r * H + 32 * grp + 8 * q + 4 * hh) = o;
      }
    }
    return;
  }
  // epilogue: lane (rr, hh) of block (mb, rb) holds y[r][m .. m + 3] for r = BR / 2 wr + 32 rb + rr and
  // m = BM / 2 wm + 32 mb + 8 q + 4 hh, q < 4
#pragma unroll
  for (int rb = 0; rb < RB; rb++) {
    const int64_t r = r0 + BR / 2 * wr + 32 * rb + rr;
    if (r >= R) continue;
#pragma unroll
    for (int mb = 0; mb < MB; mb++)
#pragma unroll
      for (int q = 0; q < 4; q++) {
        const int m = m0 + BM / 2 * wm + 32 * mb + 8 * q + 4 * hh;
        if (m >= M) continue;
        f4 v4 = f4{acc[mb][rb][4 * q], acc[mb][rb][4 * q + 1], acc[mb][rb][4 * q + 2], acc[mb][rb][4 * q + 3]};
        if (bias != nullptr) v4 += *reinterpret_cast<const f4*>(bias + m);
        TY* yp = y + r * M + m;
        if constexpr (sizeof(TY) == 4) {  // epi 1, 2 and 3 (fp32 y only)
          if (epi == 2) {
            const f4 gv = PRE ? gpre[rb][mb][q] : *reinterpret_cast<const f4*>(gate + (r % gate_rows) * ld_gate + m);
            v4 = f4{v4[0] * sigmoidf_(gv[0]), v4[1] * sigmoidf_(gv[1]), v4[2] * sigmoidf_(gv[2]),
                    v4[3] * sigmoidf_(gv[3])};
          }
          if (epi >= 1)
            v4 += PRE        ? ypre[rb][mb][q]
                  : epi == 3 ? *reinterpret_cast<const f4*>(gate + r * ld_gate + m)
                             : *reinterpret_cast<const f4*>(yp);
          *reinterpret_cast<f4*>(yp) = v4;
        } else {
          *reinterpret_cast<half4*>(yp) = half4{(half_t)v4[0], (half_t)v4[1], (half_t)v4[2], (half_t)v4[3]};
        }
      }
  }
}

// Feed-forward GEMM with the gated product in its epilogue, NP = 3: u[r][c] = silu(x[r] . Wg[c]) * (x[r] . Wx[c]) *
// (x[r] . Wab[c]) (the conditioned transition's silu(gates) * x * a_to_b, transformersv2.py:44-66); NP = 2:
// u[r][c] = silu(x[r] . W1[c]) * (x[r] . W2[c]) (Transition's SwiGLU, transition.py:27-54), without the [R, NP H]
// intermediate. W is stored in 32 NP-row groups [Wg[32 q .. +31]; Wx[..] (; Wab[..])] per 32 output columns q, so a
// workgroup tile of 32 NP W rows x 128 x rows holds all products of its 32 columns; its 4 waves own 32 x rows each
// (NP MFMA blocks of 32 x 32), and each lane ends with the NP values of 4 x 4 outputs of one row.
template <int NP>
__global__ __launch_bounds__(256, 2) void gemm_swiglu_f16_k(const half_t* __restrict__ x, const half_t* __restrict__ w,
                                                           half_t* __restrict__ u, int64_t R, int K, int H, int nr,
                                                           int nq, int per_xcd, int qfast) {
  constexpr int BM = 32 * NP, BR = 128, BK = 64, LDT = BK + 8, LA = BM / 32, LB = BR / 32;
  __shared__ LDS_ALIGN half_t As[2][BM * LDT];
  __shared__ LDS_ALIGN half_t Bs[2][BR * LDT];
  // tiles dealt to the XCDs in contiguous ranges, in the order the launcher picks (as gemm_lds_k)
  const int un = (int)(blockIdx.x % 8) * per_xcd + (int)(blockIdx.x / 8);
  if (un >= nr * nq) return;  // whole workgroup
  const int64_t r0 = (int64_t)(qfast ? un / nq : un % nr) * BR;
  const int q = qfast ? un % nq : un / nr;  // output columns 32 q .. 32 q + 31
  const int t = threadIdx.x, wave = t >> 6, l = t & 63, rr = l & 31, hh = l >> 5;
  constexpr int RSRC_CFG = 0x00020000;
  const int64_t xrows = R - r0 < BR ? R - r0 : BR;
  const __amdgpu_buffer_rsrc_t xrs =
      __builtin_amdgcn_make_buffer_rsrc((void*)(x + r0 * K), 0, (int)(xrows * K * 2), RSRC_CFG);
  const __amdgpu_buffer_rsrc_t wrs =
      __builtin_amdgcn_make_buffer_rsrc((void*)(w + (int64_t)q * BM * K), 0, (int)((int64_t)BM * K * 2), RSRC_CFG);
  const int lrow = t >> 3, lcol = (t & 7) * 8;
  u32x4_t ra0[LA], rb0[LB], ra1[LA], rb1[LB];
  auto gload = [&](u32x4_t (&ra)[LA], u32x4_t (&rb)[LB], int stage) {
#pragma unroll
    for (int v = 0; v < LA; v++) {
      const int off = (int)(((int64_t)(32 * v + lrow) * K + stage * BK + lcol) * 2);
      ra[v] = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(wrs, off, 0, 0));
    }
#pragma unroll
    for (int v = 0; v < LB; v++) {
      const int off = (int)(((int64_t)(32 * v + lrow) * K + stage * BK + lcol) * 2);
      rb[v] = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(xrs, off, 0, 0));
    }
  };
  auto lstore = [&](const u32x4_t (&ra)[LA], const u32x4_t (&rb)[LB], int buf) {
#pragma unroll
    for (int v = 0; v < LA; v++) *reinterpret_cast<u32x4_t*>(As[buf] + (32 * v + lrow) * LDT + lcol) = ra[v];
#pragma unroll
    for (int v = 0; v < LB; v++) *reinterpret_cast<u32x4_t*>(Bs[buf] + (32 * v + lrow) * LDT + lcol) = rb[v];
  };
  f16x acc[NP];
#pragma unroll
  for (int mb = 0; mb < NP; mb++)
#pragma unroll
    for (int e = 0; e < 16; e++) acc[mb][e] = 0.0f;
  auto compute = [&](int buf) {
    const half_t* Ab = As[buf] + rr * LDT + 32 * hh;
    const half_t* Bb = Bs[buf] + (32 * wave + rr) * LDT + 32 * hh;
#pragma unroll
    for (int s = 0; s < 4; s++) {
      half8 fa[NP];
#pragma unroll
      for (int mb = 0; mb < NP; mb++) fa[mb] = *reinterpret_cast<const half8*>(Ab + 32 * mb * LDT + 8 * s);
      const half8 fb = *reinterpret_cast<const half8*>(Bb + 8 * s);
#pragma unroll
      for (int mb = 0; mb < NP; mb++) acc[mb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(fa[mb], fb, acc[mb], 0, 0, 0);
    }
  };
  const int nst = K / BK;
  const int s0 = -(nst & 1);
  gload(ra0, rb0, 0);
#pragma unroll
  for (int v = 0; v < LA; v++) ra0[v] = s0 ? u32x4_t{0u, 0u, 0u, 0u} : ra0[v];
#pragma unroll
  for (int v = 0; v < LB; v++) rb0[v] = s0 ? u32x4_t{0u, 0u, 0u, 0u} : rb0[v];
  lstore(ra0, rb0, 0);
  __syncthreads();
  gload(ra0, rb0, s0 + 1);
  __builtin_amdgcn_sched_barrier(0);
  gload(ra1, rb1, min(s0 + 2, nst - 1));
  __builtin_amdgcn_sched_barrier(0);
  for (int st = s0; st < nst; st += 2) {
    compute(0);
    lstore(ra0, rb0, 1);
    __syncthreads();
    gload(ra0, rb0, min(st + 3, nst - 1));
    __builtin_amdgcn_sched_barrier(0);
    compute(1);
    lstore(ra1, rb1, 0);
    __syncthreads();
    gload(ra1, rb1, min(st + 4, nst - 1));
    __builtin_amdgcn_sched_barrier(0);
  }
  // lane (rr, hh): row r0 + 32 wave + rr, columns 32 q + 8 j + 4 hh .. + 3 in elements 4 j .. 4 j + 3 of each block
  const int64_t r = r0 + 32 * wave + rr;
  if (r >= R) return;
#pragma unroll
  for (int j = 0; j < 4; j++) {
    half4 o;
#pragma unroll
    for (int e = 0; e < 4; e++) {
      float v = siluf_(acc[0][4 * j + e]) * acc[1][4 * j + e];
      if constexpr (NP == 3) v *= acc[NP - 1][4 * j + e];
      o[e] = (half_t)v;
    }
    *reinterpret_cast<half4*>(u + r * H + 32 * q + 8 * j + 4 * hh) = o;
  }
}

template <int BM, int BR, typename TX>
hipError_t gemm_t(const void* x, const void* w, const float* bias, void* y, int y_dt, int64_t R, int K, int M,
                  int epi, const float* gate, int64_t ld_gate, int64_t gate_rows, hipStream_t st) {
  const dim3 grid((unsigned)((R + BR - 1) / BR), (unsigned)((M + BM - 1) / BM));
  if (y_dt == DT_F16)
    gemm_nt_k<BM, BR, TX, half_t><<<grid, 256, 0, st>>>(static_cast<const TX*>(x), static_cast<const TX*>(w), bias,
                                                        static_cast<half_t*>(y), R, K, M, epi, gate, ld_gate,
                                                        gate_rows);
  else
    gemm_nt_k<BM, BR, TX, float><<<grid, 256, 0, st>>>(static_cast<const TX*>(x), static_cast<const TX*>(w), bias,
                                                       static_cast<float*>(y), R, K, M, epi, gate, ld_gate,
                                                       gate_rows);
  return hipGetLastError();
}

template <int BM, int BR, int NS>
hipError_t gemm_lds_t(const void* x, const void* w, const float* bias, void* y, int y_dt, int64_t R, int K, int M,
                      int epi, const float* gate, int64_t ld_gate, int64_t gate_rows, hipStream_t st) {
  const int64_t nr = (R + BR - 1) / BR, nm = (M + BM - 1) / BM;
  if (nr * nm >= (1LL << 31) - 8 || (int64_t)(BM > BR ? BM : BR) * K * 2 > 0x7fffffffLL) return hipErrorInvalidValue;
  const int per_xcd = (int)((nr * nm + 7) / 8);
  // operand bytes one XCD reads: W tile fastest, R / 8 rows of x and all of W; x tile fastest, all of x and M / 8
  // rows of W
  const int64_t xb = R * K * 2, wb = (int64_t)M * K * 2;
  const int mfast = xb / 8 + wb <= xb + wb / 8;
  const dim3 grid((unsigned)(8 * per_xcd));
  if (y_dt == DT_F16)
    gemm_lds_k<BM, BR, NS, half_t><<<grid, 256, 0, st>>>(static_cast<const half_t*>(x), static_cast<const half_t*>(w),
                                                         bias, static_cast<half_t*>(y), R, K, M, epi, gate, ld_gate,
                                                         gate_rows, (int)nr, (int)nm, per_xcd, mfast);
  else
    gemm_lds_k<BM, BR, NS, float><<<grid, 256, 0, st>>>(static_cast<const half_t*>(x), static_cast<const half_t*>(w),
                                                        bias, static_cast<float*>(y), R, K, M, epi, gate, ld_gate,
                                                        gate_rows, (int)nr, (int)nm, per_xcd, mfast);
  return hipGetLastError();
}

// Tile choice (W rows x x rows per workgroup): 0 = 128 x 128, 1 = 128 x 64, 2 = 64 x 128, 3 = 64 x 64. The loop
// is latency-bound at these sizes (each stage's loads have two stages of compute to land), so more, smaller
// workgroups per CU win up to the 2000 x 768 x 4608 projections (64 x 64: 403-434 TF/s against 373-393 for
// 128 x 128, and 1.5-2.3x faster on the 768-wide outputs); 128 x 128 wins only on grids of thousands of its tiles
// (2000 x 768 x 36864: 454 against 378 TF/s).
int gemm_tile_choice(int64_t R, int M) {
  const int64_t n128 = ((R + 127) / 128) * ((M + 127) / 128);
  return n128 >= 2048 ? 0 : 3;
}

}  // namespace

hipError_t launch_gemm_swiglu_f16(const void* x, const void* w, void* u, int64_t R, int K, int H, int np,
                                  hipStream_t st) {
  const auto al = [](const void* p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0; };
  if (R < 1 || K % 64 || K < 64 || H % 32 || H < 32 || (int64_t)128 * K * 2 > 0x7fffffffLL || !al(x, 16) ||
      !al(w, 16) || !al(u, 8) || (R + 127) / 128 > 0x7fffffffLL || (np != 2 && np != 3))
    return hipErrorInvalidValue;
  const int64_t xb = R * K * 2, wb = (int64_t)np * H * K * 2;
  // 2048 rows and more, H a multiple of 64: the LDS-direct tiles (64 np W rows = two column groups x 128 rows, two
  // stages, two workgroups per CU; the diffusion transformer's 2000 x 768 -> 3 x 1536 in one round of 384 tiles)
  if (R >= 1536 && H % 64 == 0) {
    const int64_t nr = (R + 127) / 128, nm = H / 64;
    if (nr * nm >= (1LL << 31) - 8 || (int64_t)64 * np * K * 2 > 0x7fffffffLL) return hipErrorInvalidValue;
    const int per_xcd = (int)((nr * nm + 7) / 8), mfast = xb / 8 + wb <= xb + wb / 8;
    const dim3 grid((unsigned)(8 * per_xcd));
    if (np == 3)
      gemm_lds_k<192, 128, 2, half_t, 3><<<grid, 256, 0, st>>>(
          static_cast<const half_t*>(x), static_cast<const half_t*>(w), nullptr, static_cast<half_t*>(u), R, K, 3 * H,
          0, nullptr, 0, 1, (int)nr, (int)nm, per_xcd, mfast);
    else
      gemm_lds_k<128, 128, 2, half_t, 2><<<grid, 256, 0, st>>>(
          static_cast<const half_t*>(x), static_cast<const half_t*>(w), nullptr, static_cast<half_t*>(u), R, K, 2 * H,
          0, nullptr, 0, 1, (int)nr, (int)nm, per_xcd, mfast);
    return hipGetLastError();
  }
  const int64_t nr = (R + 127) / 128, nq = H / 32;
  if (nr * nq >= (1LL << 31) - 8) return hipErrorInvalidValue;
  const int per_xcd = (int)((nr * nq + 7) / 8);
  const int qfast = xb / 8 + wb <= xb + wb / 8;
  const dim3 grid((unsigned)(8 * per_xcd));
  if (np == 3)
    gemm_swiglu_f16_k<3><<<grid, 256, 0, st>>>(static_cast<const half_t*>(x), static_cast<const half_t*>(w),
                                               static_cast<half_t*>(u), R, K, H, (int)nr, (int)nq, per_xcd, qfast);
  else
    gemm_swiglu_f16_k<2><<<grid, 256, 0, st>>>(static_cast<const half_t*>(x), static_cast<const half_t*>(w),
                                               static_cast<half_t*>(u), R, K, H, (int)nr, (int)nq, per_xcd, qfast);
  return hipGetLastError();
}

bool gemm_nt_ok(int x_dt, const void* x, const void* w, const float* bias, const void* y, int64_t R, int K, int M,
                const float* gate, int64_t ld_gate) {
  const auto al = [](const void* p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0; };
  const int es = x_dt == DT_F16 ? 2 : 4;
  return K % (128 / es) == 0 && M % 4 == 0 && R >= 1 && (int64_t)128 * K * es <= 0x7fffffffLL && al(x, 16) &&
         al(w, 16) && al(y, 16) && (bias == nullptr || al(bias, 16)) &&
         (gate == nullptr || (al(gate, 16) && ld_gate % 4 == 0));
}

hipError_t launch_gemm_nt(const void* x, const void* w, const float* bias, void* y, int x_dt, int y_dt, int64_t R,
                          int K, int M, int epi, const float* gate, int64_t ld_gate, int64_t gate_rows,
                          hipStream_t st) {
  if ((x_dt != DT_F16 && x_dt != DT_F32) || !gemm_nt_ok(x_dt, x, w, bias, y, R, K, M, gate, ld_gate) || epi < 0 ||
      epi > 3 || (epi >= 1 && y_dt != DT_F32) || (epi >= 2 && (gate == nullptr || gate_rows < 1)))
    return hipErrorInvalidValue;
  if (x_dt == DT_F32)  // fp32 operands: 64 x 64 tiles (the m track's 409,600-row projections)
    return gemm_t<64, 64, float>(x, w, bias, y, y_dt, R, K, M, epi, gate, ld_gate, gate_rows, st);
  // below the large-grid case, for 2048 rows and more, the LDS-direct form with 3 stages (2 in flight) takes the
  // same tiles: the diffusion transformer's 2000 x 768 -> 3072 projection 24.4 -> 22.1 us (128 x 64), its 768-wide
  // gated outputs 12.6 -> 11.7 and 17.2 -> 16.1 us (64 x 64). Same sums in the same order. The s track's GEMMs
  // (N rows) keep the register-staged form: they run beside the attention core, and there the LDS-direct form's
  // workgroups found compute units far later (0.85 ms against 0.04 ms per launch at N = 1000).
  // 128 columns over many rows (the outer product mean's proj_o, 160,000 x 1024 -> 128 at N = 400): one 128-wide
  // column tile, so each x row is read once (124.8 against 148.0 us on 64 x 64 tiles; 128 x 64 and 64 x 128 with
  // three stages 130.5 and 129.0)
  if (M == 128 && R >= 65536)
    return gemm_lds_t<128, 128, 2>(x, w, bias, y, y_dt, R, K, M, epi, gate, ld_gate, gate_rows, st);
  if (gemm_tile_choice(R, M) != 0 && R >= 1536)
    return M >= 2048 ? gemm_lds_t<192, 128, 3>(x, w, bias, y, y_dt, R, K, M, epi, gate, ld_gate, gate_rows, st)
                     : gemm_lds_t<64, 64, 3>(x, w, bias, y, y_dt, R, K, M, epi, gate, ld_gate, gate_rows, st);
  switch (gemm_tile_choice(R, M)) {
    case 0: return gemm_t<128, 128, half_t>(x, w, bias, y, y_dt, R, K, M, epi, gate, ld_gate, gate_rows, st);
    case 1: return gemm_t<128, 64, half_t>(x, w, bias, y, y_dt, R, K, M, epi, gate, ld_gate, gate_rows, st);
    case 2: return gemm_t<64, 128, half_t>(x, w, bias, y, y_dt, R, K, M, epi, gate, ld_gate, gate_rows, st);
    default: return gemm_t<64, 64, half_t>(x, w, bias, y, y_dt, R, K, M, epi, gate, ld_gate, gate_rows, st);
  }
}

}  // namespace bzpf
