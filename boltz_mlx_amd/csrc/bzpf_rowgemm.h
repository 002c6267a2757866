// Transposed row-tile GEMM building blocks for the pair kernels (K = 128 input channels per row).
//
// The kernels compute Y^T = W X^T on MFMA: A = a 16-row block of the weight W (output channels, K-contiguous, staged
// in LDS), B = X^T for 16 rows of X (positions, K-contiguous, loaded once per tile straight from global memory into
// registers). The accumulator then holds, per lane l, row l % 16 of X and the 4 consecutive output channels
// 16*cb + 4*(l/16) + e, e = 0..3: every row lives in 4 lanes (l, l^16, l^32, l^48), so row-wise epilogues (residual
// add, LayerNorm) need two cross-lane steps, and each lane writes 4 contiguous outputs.
// K is split in lane-group blocks: MFMA step s of lane group g = l/16 takes k = 32*g + s*KP + t (t < KP), which is a
// permutation of the sum over k shared by A and B, so a lane reads 32 contiguous channels of its row.
#pragma once

#include "bzpf_common.h"

namespace bzpf {

template <typename T> struct RG;
template <> struct RG<half_t> {
  static constexpr int STEPS = 4;  // MFMA steps over K = 128
  typedef half8 frag;
  __device__ static __forceinline__ void load_row(frag (&f)[STEPS], const half_t* p, int g) {
#pragma unroll
    for (int s = 0; s < STEPS; s++) f[s] = *reinterpret_cast<const half8*>(p + 32 * g + 8 * s);
  }
  __device__ static __forceinline__ void zero(frag (&f)[STEPS]) {
#pragma unroll
    for (int s = 0; s < STEPS; s++)
#pragma unroll
      for (int t = 0; t < 8; t++) f[s][t] = (half_t)0.0f;
  }
};
template <> struct RG<float> {
  static constexpr int STEPS = 32;
  typedef float frag;
  __device__ static __forceinline__ void load_row(frag (&f)[STEPS], const float* p, int g) {
#pragma unroll
    for (int j = 0; j < 8; j++) {
      const f4 v = *reinterpret_cast<const f4*>(p + 32 * g + 4 * j);
      f[4 * j] = v[0]; f[4 * j + 1] = v[1]; f[4 * j + 2] = v[2]; f[4 * j + 3] = v[3];
    }
  }
  __device__ static __forceinline__ void zero(frag (&f)[STEPS]) {
#pragma unroll
    for (int s = 0; s < STEPS; s++) f[s] = 0.0f;
  }
};

// Row blocks per wave: fp16 tiles are 128 rows per workgroup (2 blocks per wave), fp32 tiles 64 rows.
template <typename T> struct RowBlocks { static constexpr int v = sizeof(T) == 2 ? 2 : 1; };

// acc[rb][cb] += W[16 cb .. +15][0:128] . X[rb]^T for CB column blocks of the LDS weight chunk Ws (pitch ldw).
// ROWS = true computes the same block untransposed, acc[rb][cb] += X[rb] . W[16 cb .. +15]^T: the two operand
// layouts of the MFMA are mirror images (lane l holds 8 k-consecutive elements of row/column l % 16), so swapping
// the operands swaps the accumulator layout. Then lane l holds rows (positions) 4 (l/16) + e of block rb and output
// channel 16 cb + l % 16: position-contiguous runs, for outputs stored channel-major.
template <typename T, int RB, int CB, bool ROWS = false>
__device__ __forceinline__ void mma_rows(f4 (&acc)[RB][CB], const typename RG<T>::frag (&x)[RB][RG<T>::STEPS],
                                         const T* Ws, int ldw) {
  const int l = threadIdx.x & 63, g = l >> 4;
#pragma unroll
  for (int cb = 0; cb < CB; cb++) {
    const T* wp = Ws + (16 * cb + (l & 15)) * ldw + 32 * g;
    if constexpr (sizeof(T) == 2) {
#pragma unroll
      for (int s = 0; s < 4; s++) {
        const half8 a = *reinterpret_cast<const half8*>(wp + 8 * s);
#pragma unroll
        for (int rb = 0; rb < RB; rb++)
          acc[rb][cb] = ROWS ? __builtin_amdgcn_mfma_f32_16x16x32_f16(x[rb][s], a, acc[rb][cb], 0, 0, 0)
                             : __builtin_amdgcn_mfma_f32_16x16x32_f16(a, x[rb][s], acc[rb][cb], 0, 0, 0);
      }
    } else {
#pragma unroll
      for (int j = 0; j < 8; j++) {
        const f4 a = *reinterpret_cast<const f4*>(wp + 4 * j);
#pragma unroll
        for (int t = 0; t < 4; t++)
#pragma unroll
          for (int rb = 0; rb < RB; rb++)
            acc[rb][cb] = ROWS ? __builtin_amdgcn_mfma_f32_16x16x4f32(x[rb][4 * j + t], a[t], acc[rb][cb], 0, 0, 0)
                               : __builtin_amdgcn_mfma_f32_16x16x4f32(a[t], x[rb][4 * j + t], acc[rb][cb], 0, 0, 0);
      }
    }
  }
}

// Position tiles for channel-major outputs (ROWS orientation): a wave tile is TW = 16 RB positions, and the row that
// lane r (= l % 16) loads for row block rb is position pos(rb, r) = 4 RB (r / 4) + 4 rb + r % 4. The accumulator
// lane of group g then holds positions 4 RB g .. 4 RB g + 4 RB - 1 (index 4 rb + e) of one channel: 16 bytes of T.
template <typename T> struct RunTile {
  static constexpr int RB = sizeof(T) == 2 ? 2 : 1;
  static constexpr int TW = 16 * RB;
  static constexpr int RUN = 4 * RB;
  __device__ static __forceinline__ int pos(int rb, int r) { return RUN * (r >> 2) + 4 * rb + (r & 3); }
};

// Store RUN = 16 / sizeof(T) consecutive values as one 16-byte vector. The projections' outputs are streamed once and
// read back by the next kernel, so the stores are non-temporal (measured: the attention projection's q/k/g/V^T
// writes run 20% faster than through the default cache policy).
__device__ __forceinline__ void st_run(half_t* p, const float (&v)[8]) {
  __builtin_nontemporal_store(half8{(half_t)v[0], (half_t)v[1], (half_t)v[2], (half_t)v[3], (half_t)v[4],
                                    (half_t)v[5], (half_t)v[6], (half_t)v[7]},
                              reinterpret_cast<half8*>(p));
}
__device__ __forceinline__ void st_run(float* p, const float (&v)[4]) {
  __builtin_nontemporal_store(f4{v[0], v[1], v[2], v[3]}, reinterpret_cast<f4*>(p));
}
// The same runs through the default cache policy (the trimul projection: its half-line runs of one channel row
// merge in L2 before they are written back; measured 7-10% faster there than non-temporal stores).
__device__ __forceinline__ void st_run_cached(half_t* p, const float (&v)[8]) {
  *reinterpret_cast<half8*>(p) = half8{(half_t)v[0], (half_t)v[1], (half_t)v[2], (half_t)v[3], (half_t)v[4],
                                       (half_t)v[5], (half_t)v[6], (half_t)v[7]};
}
__device__ __forceinline__ void st_run_cached(float* p, const float (&v)[4]) {
  *reinterpret_cast<f4*>(p) = f4{v[0], v[1], v[2], v[3]};
}

// mma_rows over CB column blocks in groups of G with a scheduling barrier between groups: the compiler otherwise
// hoists every LDS weight read ahead of the MFMAs (CB * 4 fragments live at once), which spills at 4 waves/SIMD.
template <typename T, int RB, int CB, int G, bool ROWS = false>
__device__ __forceinline__ void mma_rows_grouped(f4 (&acc)[RB][CB], const typename RG<T>::frag (&x)[RB][RG<T>::STEPS],
                                                 const T* Ws, int ldw) {
  static_assert(CB % G == 0, "column blocks must split into groups");
#pragma unroll
  for (int q = 0; q < CB / G; q++) {
    f4 part[RB][G];
#pragma unroll
    for (int rb = 0; rb < RB; rb++)
#pragma unroll
      for (int c = 0; c < G; c++) part[rb][c] = acc[rb][G * q + c];
    mma_rows<T, RB, G, ROWS>(part, x, Ws + 16 * G * q * ldw, ldw);
#pragma unroll
    for (int rb = 0; rb < RB; rb++)
#pragma unroll
      for (int c = 0; c < G; c++) acc[rb][G * q + c] = part[rb][c];
    __builtin_amdgcn_sched_barrier(0);
  }
}

// Copy `rows` rows of `k` elements (k % (16 / sizeof(T)) == 0) into LDS [rows][ld]; row r comes from src(r)
// (nullptr: zeros).
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

template <typename T, typename RowFn>
__device__ __forceinline__ void lds_rows(T* dst, int ld, int rows, int k, RowFn src) {
  constexpr int VE = 16 / sizeof(T);
  const int per = k / VE;
  for (int e = threadIdx.x; e < rows * per; e += blockDim.x) {
    const int r = e / per, c = (e - r * per) * VE;
    const T* s = src(r);
    u32x4 v = u32x4{0u, 0u, 0u, 0u};
    if (s) v = *reinterpret_cast<const u32x4*>(s + c);
    *reinterpret_cast<u32x4*>(dst + r * ld + c) = v;
  }
}

// LayerNorm weight and bias (128 channels each) staged in LDS for the epilogues below, which read them per 16-channel
// block. From global memory each of those reads is a separate round trip whose s_waitcnt vmcnt(0) also waits for
// every tile prefetch and store issued before it (the counter is in order), once per column block; from LDS they
// are lgkmcnt waits only. stage_ln runs before the kernel's first barrier; w == nullptr leaves the arrays unset.
struct LnLds {
  float w[128];
  float b[128];
};
__device__ __forceinline__ void stage_ln(LnLds& s, const float* __restrict__ w, const float* __restrict__ b) {
  if (w == nullptr) return;
  for (int c = threadIdx.x; c < 128; c += blockDim.x) {
    s.w[c] = w[c];
    s.b[c] = b[c];
  }
}

// 4 consecutive elements of T from / to memory as fp32.
__device__ __forceinline__ f4 ld4(const float* p) { return *reinterpret_cast<const f4*>(p); }
__device__ __forceinline__ f4 ld4(const half_t* p) {
  const half4 h = *reinterpret_cast<const half4*>(p);
  return f4{(float)h[0], (float)h[1], (float)h[2], (float)h[3]};
}
__device__ __forceinline__ void st4(float* p, f4 v) { *reinterpret_cast<f4*>(p) = v; }
__device__ __forceinline__ void st4(half_t* p, f4 v) {
  *reinterpret_cast<half4*>(p) = half4{(half_t)v[0], (half_t)v[1], (half_t)v[2], (half_t)v[3]};
}

// The residual rows the epilogue below adds to, in the accumulator layout (lane: 4 channels 16 cb + 4 g .. +3 of its
// row); zeros where accumulate == 0. A lane with no row (zrow < 0) loads row 0 instead: its values only enter the
// reductions of its own row, which is never stored, and the loads stay unconditional (no per-lane branches).
// Issued ahead of the MFMAs so the loads overlap them.
template <int RB, typename ZRow>
__device__ __forceinline__ void load_z_rows(f4 (&zv)[RB][8], ZRow zrow, const float* __restrict__ z, int accumulate) {
  constexpr int D = 128;
  const int g = (threadIdx.x & 63) >> 4;
#pragma unroll
  for (int rb = 0; rb < RB; rb++) {
    const int64_t zr = zrow(rb);
    const float* zp = z + (zr >= 0 ? zr : 0) * D + 4 * g;  // one row base; column blocks are immediate offsets
#pragma unroll
    for (int cb = 0; cb < 8; cb++) zv[rb][cb] = accumulate ? ld4(zp + 16 * cb) : f4{0.f, 0.f, 0.f, 0.f};
  }
}

// Residual + LayerNorm epilogue on the transposed accumulator of 8 column blocks (D = 128 channels): for each of the
// lane's rows, z[zr] = zv + y, then xn_next[zr] = LN(z[zr]) when lnw != nullptr. zrow(rb) returns the z row of the
// lane's row in block rb (< 0: no row; the lane still joins the cross-lane reductions, which only mix the 4 lanes
// of one row, and stores nothing).
template <typename TO, int RB, typename ZRow>
__device__ __forceinline__ void resid_ln_apply(const f4 (&y)[RB][8], const f4 (&zv)[RB][8], ZRow zrow,
                                               float* __restrict__ z, const float* __restrict__ lnw,
                                               const float* __restrict__ lnb, float eps, TO* __restrict__ xn_next) {
  constexpr int D = 128;
  const int l = threadIdx.x & 63, g = l >> 4;
#pragma unroll
  for (int rb = 0; rb < RB; rb++) {
    const int64_t zr = zrow(rb);
    // one row base per pointer; the column blocks 16 cb are immediate offsets (no per-block 64-bit addresses)
    const int64_t rowoff = (zr >= 0 ? zr : 0) * D + 4 * g;
    float* zp = z + rowoff;
    f4 v[8];
    float s = 0.f;
#pragma unroll
    for (int cb = 0; cb < 8; cb++) {
      v[cb] = y[rb][cb] + zv[rb][cb];
      s += v[cb][0] + v[cb][1] + v[cb][2] + v[cb][3];
    }
    if (zr >= 0) {
#pragma unroll
      for (int cb = 0; cb < 8; cb++) __builtin_nontemporal_store(v[cb], reinterpret_cast<f4*>(zp + 16 * cb));
    }
    if (lnw == nullptr) continue;
    const float mean = xgroups_sum(s) * (1.0f / D);
    float ss = 0.f;
#pragma unroll
    for (int cb = 0; cb < 8; cb++) {
      const f4 d = v[cb] - mean;
      ss += d[0] * d[0] + d[1] * d[1] + d[2] * d[2] + d[3] * d[3];
    }
    const float rstd = 1.0f / sqrtf(xgroups_sum(ss) * (1.0f / D) + eps);
    if (zr < 0) continue;
    TO* xp = xn_next + rowoff;
#pragma unroll
    for (int cb = 0; cb < 8; cb++) {
      const int c = 16 * cb + 4 * g;
      st4(xp + 16 * cb, (v[cb] - mean) * rstd * ld4(lnw + c) + ld4(lnb + c));
    }
  }
}

// z[zr] = (accumulate ? z[zr] : 0) + y, then the next LayerNorm (resid_ln_apply with the residual loaded in place).
template <typename TO, int RB, typename ZRow>
__device__ __forceinline__ void resid_ln_rows(const f4 (&y)[RB][8], ZRow zrow, float* __restrict__ z, int accumulate,
                                              const float* __restrict__ lnw, const float* __restrict__ lnb, float eps,
                                              TO* __restrict__ xn_next) {
  f4 zv[RB][8];
  load_z_rows<RB>(zv, zrow, z, accumulate);
  resid_ln_apply<TO, RB>(y, zv, zrow, z, lnw, lnb, eps, xn_next);
}

// The triangle attention's output stage run in front of a fused transition, on RB row blocks of 16 rows: y = W_o o^T
// (x holds the o rows as B fragments, W_o [128][ldw] in LDS), z' = z[zr] + y, then x <- LN(z') in fp16 as B
// fragments again (the transition's input). z' is not stored: the epilogue recomputes it (the same MFMA order,
// so the same bits) rather than reading back a copy. The LayerNorm output leaves the accumulator layout
// (lane: 4 channels of each 16-channel block) through a wave-private LDS scratch of 16 rows (pitch SCR_P halves),
// written and read back by the same wave in program order, so it needs no barrier; the arithmetic is
// resid_ln_apply's, so x equals the fp16 rows that kernel would have written.
constexpr int SCR_P = 144;
template <int RB, typename ZRow>
__device__ __forceinline__ void attn_out_rows(RG<half_t>::frag (&x)[RB][4], const half_t* Wo, int ldw, ZRow zrow,
                                              const float* __restrict__ z, const float* __restrict__ lnw,
                                              const float* __restrict__ lnb, float eps, half_t* scr) {
  constexpr int D = 128;
  const int l = threadIdx.x & 63, g = l >> 4, r = l & 15;
  f4 y[RB][8];
  zero_acc(y);
  mma_rows_grouped<half_t, RB, 8, 2>(y, x, Wo, ldw);
  f4 zv[RB][8];
  load_z_rows<RB>(zv, zrow, z, 1);
#pragma unroll
  for (int rb = 0; rb < RB; rb++) {
    f4 v[8];
    float s = 0.f;
#pragma unroll
    for (int cb = 0; cb < 8; cb++) {
      v[cb] = y[rb][cb] + zv[rb][cb];
      s += v[cb][0] + v[cb][1] + v[cb][2] + v[cb][3];
    }
    const float mean = xgroups_sum(s) * (1.0f / D);
    float ss = 0.f;
#pragma unroll
    for (int cb = 0; cb < 8; cb++) {
      const f4 d = v[cb] - mean;
      ss += d[0] * d[0] + d[1] * d[1] + d[2] * d[2] + d[3] * d[3];
    }
    const float rstd = 1.0f / sqrtf(xgroups_sum(ss) * (1.0f / D) + eps);
    half_t* sw = scr + r * SCR_P + 4 * g;
#pragma unroll
    for (int cb = 0; cb < 8; cb++) {
      const int c = 16 * cb + 4 * g;
      st4(sw + 16 * cb, (v[cb] - mean) * rstd * ld4(lnw + c) + ld4(lnb + c));
    }
    RG<half_t>::load_row(x[rb], scr + r * SCR_P, g);
  }
}

// resid_ln_rows for fp16 rows, plus the pair bias Linear(LN_pb(z_new)) of the s track from the same row statistics:
// with W' = W ⊙ gamma_pb (fp16, LDS [16][ldp]) and bp = W . beta_pb (LDS, fp32),
//   pb_out[h][zr] = (x_hat . W'[h]) + bp[h],  x_hat = (z_new - mean) * rstd_pb,
// on one v_mfma_f32_16x16x32_f16 per 32 channels: the B operand is the lane's own 32 normalised channels of its row
// (k slot 8 g + t <-> channel 32 s + 16 (t / 4) + 4 g + t % 4 in step s), A the same channels of W' for head l % 16,
// and the accumulator lane (row, g) receives heads 4 g .. 4 g + 3 of its row. The MFMAs run with every lane active;
// lanes without a row compute on finite stand-in values and store nothing.
// resid_ln_pb_apply takes the residual rows from zvf(rb, zv) (zv: the row block's 8 column blocks, accumulator
// layout); resid_ln_pb_rows loads them from z first.
template <int RB, typename ZRow, typename ZvFn>
__device__ __forceinline__ void resid_ln_pb_apply(const f4 (&y)[RB][8], ZvFn zvf, ZRow zrow, float* __restrict__ z,
                                                  const float* __restrict__ lnw, const float* __restrict__ lnb,
                                                  float eps, half_t* __restrict__ xn_next, const half_t* Wp, int ldp,
                                                  const float* Bp, float eps_pb, half_t* __restrict__ pb_out,
                                                  int64_t pb_stride, int pb_heads) {
  constexpr int D = 128;
  const int l = threadIdx.x & 63, g = l >> 4, r = l & 15;
#pragma unroll
  for (int rb = 0; rb < RB; rb++) {
    f4 zv[8];
    zvf(rb, zv);
    const int64_t zr = zrow(rb);
    const int64_t rowoff = (zr >= 0 ? zr : 0) * D + 4 * g;
    float* zp = z + rowoff;
    f4 v[8];
    float s = 0.f;
#pragma unroll
    for (int cb = 0; cb < 8; cb++) {
      v[cb] = y[rb][cb] + zv[cb];
      s += v[cb][0] + v[cb][1] + v[cb][2] + v[cb][3];
    }
    if (zr >= 0) {
#pragma unroll
      for (int cb = 0; cb < 8; cb++) __builtin_nontemporal_store(v[cb], reinterpret_cast<f4*>(zp + 16 * cb));
    }
    const float mean = xgroups_sum(s) * (1.0f / D);
    float ss = 0.f;
#pragma unroll
    for (int cb = 0; cb < 8; cb++) {
      const f4 d = v[cb] - mean;
      ss += d[0] * d[0] + d[1] * d[1] + d[2] * d[2] + d[3] * d[3];
    }
    const float var = xgroups_sum(ss) * (1.0f / D);
    if (lnw != nullptr && zr >= 0) {
      const float rstd = 1.0f / sqrtf(var + eps);
      half_t* xp = xn_next + rowoff;
#pragma unroll
      for (int cb = 0; cb < 8; cb++) {
        const int c = 16 * cb + 4 * g;
        st4(xp + 16 * cb, (v[cb] - mean) * rstd * ld4(lnw + c) + ld4(lnb + c));
      }
    }
    const float rpb = 1.0f / sqrtf(var + eps_pb);
    f4 acc = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int st = 0; st < 4; st++) {
      const f4 lo = (v[2 * st] - mean) * rpb, hi = (v[2 * st + 1] - mean) * rpb;
      const half8 bf = half8{(half_t)lo[0], (half_t)lo[1], (half_t)lo[2], (half_t)lo[3],
                             (half_t)hi[0], (half_t)hi[1], (half_t)hi[2], (half_t)hi[3]};
      const half_t* wr = Wp + r * ldp + 32 * st + 4 * g;
      const half4 wlo = *reinterpret_cast<const half4*>(wr);
      const half4 whi = *reinterpret_cast<const half4*>(wr + 16);
      const half8 af = half8{wlo[0], wlo[1], wlo[2], wlo[3], whi[0], whi[1], whi[2], whi[3]};
      acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(af, bf, acc, 0, 0, 0);
    }
    if (zr >= 0) {
#pragma unroll
      for (int e = 0; e < 4; e++) {
        const int h = 4 * g + e;
        if (h < pb_heads) pb_out[(int64_t)h * pb_stride + zr] = (half_t)(acc[e] + Bp[h]);
      }
    }
  }
}

template <int RB, typename ZRow>
__device__ __forceinline__ void resid_ln_pb_rows(const f4 (&y)[RB][8], ZRow zrow, float* __restrict__ z, int accumulate,
                                                 const float* __restrict__ lnw, const float* __restrict__ lnb,
                                                 float eps, half_t* __restrict__ xn_next, const half_t* Wp, int ldp,
                                                 const float* Bp, float eps_pb, half_t* __restrict__ pb_out,
                                                 int64_t pb_stride, int pb_heads) {
  f4 zv[RB][8];
  load_z_rows<RB>(zv, zrow, z, accumulate);
  resid_ln_pb_apply<RB>(
      y,
      [&](int rb, f4(&o)[8]) {
#pragma unroll
        for (int cb = 0; cb < 8; cb++) o[cb] = zv[rb][cb];
      },
      zrow, z, lnw, lnb, eps, xn_next, Wp, ldp, Bp, eps_pb, pb_out, pb_stride, pb_heads);
}

// Index of the calling wave in the grid as a wave-uniform (scalar) value: the compiler cannot prove threadIdx.x / 64
// uniform by itself, and tile coordinates derived from it would otherwise live (and be divided) in vector registers.
__device__ __forceinline__ int grid_wave(int waves_per_block) {
  return __builtin_amdgcn_readfirstlane((int)(blockIdx.x * waves_per_block + (threadIdx.x >> 6)));
}

// Persistent launches: each wave walks tiles wave_id, wave_id + waves_in_grid, ... so the grid is sized to what stays
// resident (resident workgroups per CU x CUs) and the weights staged in LDS once per workgroup serve all its tiles.
// `cache` holds the answer per device (0: not yet queried); returns 0 if the runtime cannot answer.
constexpr int kMaxDevices = 64;
template <typename Kern>
static int resident_grid(Kern kernel, int threads, int (&cache)[kMaxDevices]) {
  int dev = 0, cus = 0, per = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0) return 0;
  if (dev < kMaxDevices && cache[dev] > 0) return cache[dev];
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per, kernel, threads, 0) != hipSuccess) return 0;
  const int n = cus * (per > 0 ? per : 1);
  if (dev < kMaxDevices) cache[dev] = n;
  return n;
}

}  // namespace bzpf
