// The MSA track's input projection, LayerNorm and Linear in one kernel at fp32 accuracy:
//   y[r][m] = LN(x[r]; ln_w, ln_b, eps) . W[m]   for fp32 x [R, 64], W [M, 64] (M a multiple of 256), y [R, M]
// (PairWeightedAveraging's norm_m + proj_m | proj_g, boltz_mlx/layers/pair_averaging.py:36-41, fp32 in both
// precision modes). The LayerNorm is the arithmetic of bzpf_layernorm (16 lanes per row, the same sums), so its
// output is the same fp32 values; the product runs on the bf16 matrix cores with both operands split into three
// exact bf16 parts (bzpf_x3.h). The projection has K = 64 and writes M fp32 values per row, so it is bound by its
// stores: the kernel is persistent, one 8-wave workgroup per CU, with a 256-column block of W split into LDS once,
// and each 128-row tile's x rows loaded while the previous tile computes and stores.
#include "bzpf_common.h"
#include "bzpf_kernels.h"
#include "bzpf_rowgemm.h"
#include "bzpf_x3.h"

namespace bzpf {

namespace {

constexpr int LNP_K = 64, LNP_BR = 128, LNP_BC = 256;  // channels; the largest row and column tiles
constexpr int LNP_ROWB = 2 * LNP_K;                    // bytes of one plane row (64 bf16)

// Byte offset of 16-byte chunk c (k = 8 c .. 8 c + 7) of plane row r: the chunks of a row are permuted by r % 8, so
// the fragment reads (8 lanes on 8 consecutive rows at one logical chunk) hit distinct banks.
__device__ __forceinline__ int lnp_off(int r, int c) { return r * LNP_ROWB + 16 * (c ^ (r & 7)); }

// Workgroup b takes column block cb = b % ncb and the row tiles b / ncb, b / ncb + gridDim.x / ncb, ... of BR rows
// against BC columns; wave (wr, wc) = (wave / WC, wave % WC) computes rows BR / WR wr .. x columns BC / WC wc .. of
// the tile (MB x NB blocks of 32 x 32).
template <int BR, int BC, int WR, int WC>
__global__ __launch_bounds__(64 * WR * WC, 8 / (WR * WC)) void ln_linear_x3_k(const float* __restrict__ x,
                                                                 const float* __restrict__ lnw,
                                                                 const float* __restrict__ lnb, float eps,
                                                                 const float* __restrict__ w, float* __restrict__ y,
                                                                 int64_t R, int M, int ncb, int nrt) {
  constexpr int NT = 64 * WR * WC, MB = BR / WR / 32, NB = BC / WC / 32;
  constexpr int XP = BR * 16 / NT, WP = BC * 16 / NT;  // x rows per thread, W f4 items per thread
  static_assert(MB >= 1 && NB >= 1 && XP >= 1 && WP >= 1, "tile shape");
  __shared__ __attribute__((aligned(16))) char Ws[3 * BC * LNP_ROWB];  // the W block's three planes
  __shared__ __attribute__((aligned(16))) char Xs[3 * BR * LNP_ROWB];  // the tile's LN(x) planes
  const int t = threadIdx.x, wave = t >> 6, l = t & 63, r32 = l & 31, hl = l >> 5;
  const int wr = wave / WC, wc = wave % WC;
  const int cb = (int)blockIdx.x % ncb, m0 = cb * BC;
  // the W block, split once: f4 item e = t + NT v is row e / 16 (clamped to M - 1), k = 4 (e % 16) .. + 3
#pragma unroll
  for (int v = 0; v < WP; v++) {
    const int e = t + NT * v, row = e >> 4, kq = e & 15;
    const f4 a = *reinterpret_cast<const f4*>(w + (int64_t)min(m0 + row, M - 1) * LNP_K + 4 * kq);
    const Pair3 q01 = split3_pair(a[0], a[1]), q23 = split3_pair(a[2], a[3]);
#pragma unroll
    for (int p = 0; p < 3; p++)
      *reinterpret_cast<uint2*>(Ws + p * BC * LNP_ROWB + lnp_off(row, kq >> 1) + 8 * (kq & 1)) =
          uint2{q01.p[p], q23.p[p]};
  }
  // x rows: pass v takes tile row t / 16 + NT / 16 v, lane c = t % 16 channels 4 c .. + 3 (rows past R read row
  // R - 1; their outputs are not stored)
  const int xc = t & 15, xrow = t >> 4;
  const f4 gw = *reinterpret_cast<const f4*>(lnw + 4 * xc), gb = *reinterpret_cast<const f4*>(lnb + 4 * xc);
  f4 xv[XP];
  auto xload = [&](int rt) {
#pragma unroll
    for (int v = 0; v < XP; v++) {
      const int64_t r = min((int64_t)rt * BR + xrow + NT / 16 * v, R - 1);
      xv[v] = *reinterpret_cast<const f4*>(x + r * LNP_K + 4 * xc);
    }
  };
  // LN (bzpf_layernorm's order of operations), then the split into the X planes
  auto xstage = [&]() {
#pragma unroll
    for (int v = 0; v < XP; v++) {
      const f4 a = xv[v];
      float s = 0.f;
      s += a[0] + a[1] + a[2] + a[3];
      const float mean = group_sum<16>(s) * (1.0f / LNP_K);
      float ss = 0.f;
      const f4 d = a - mean;
      ss += d[0] * d[0] + d[1] * d[1] + d[2] * d[2] + d[3] * d[3];
      const float rstd = 1.0f / sqrtf(group_sum<16>(ss) * (1.0f / LNP_K) + eps);
      f4 o = (a - mean) * rstd;
      o *= gw;
      o += gb;
      const Pair3 q01 = split3_pair(o[0], o[1]), q23 = split3_pair(o[2], o[3]);
      const int row = xrow + NT / 16 * v;
#pragma unroll
      for (int p = 0; p < 3; p++)
        *reinterpret_cast<uint2*>(Xs + p * BR * LNP_ROWB + lnp_off(row, xc >> 1) + 8 * (xc & 1)) =
            uint2{q01.p[p], q23.p[p]};
    }
  };
  const int rstep = (int)gridDim.x / ncb;
  int rt = (int)blockIdx.x / ncb;
  if (rt < nrt) xload(rt);
  for (; rt < nrt; rt += rstep) {  // workgroup-uniform
    xstage();
    __syncthreads();  // the X planes (and, the first time, the W planes) are complete
    if (rt + rstep < nrt) xload(rt + rstep);
    f16x acc[MB][NB];
#pragma unroll
    for (int a = 0; a < MB; a++)
#pragma unroll
      for (int b = 0; b < NB; b++)
#pragma unroll
        for (int e = 0; e < 16; e++) acc[a][b][e] = 0.0f;
#pragma unroll
    for (int kk = 0; kk < LNP_K / 16; kk++) {
      bf16x8 fa[MB][3], fb[NB][3];
#pragma unroll
      for (int bm = 0; bm < MB; bm++)
#pragma unroll
        for (int p = 0; p < 3; p++)
          fa[bm][p] = *reinterpret_cast<const bf16x8*>(Xs + p * BR * LNP_ROWB +
                                                       lnp_off(BR / WR * wr + 32 * bm + r32, 2 * kk + hl));
#pragma unroll
      for (int bn = 0; bn < NB; bn++)
#pragma unroll
        for (int p = 0; p < 3; p++)
          fb[bn][p] = *reinterpret_cast<const bf16x8*>(Ws + p * BC * LNP_ROWB +
                                                       lnp_off(BC / WC * wc + 32 * bn + r32, 2 * kk + hl));
#pragma unroll
      for (int bm = 0; bm < MB; bm++)
#pragma unroll
        for (int bn = 0; bn < NB; bn++) acc[bm][bn] = mfma_parts6(fa[bm], fb[bn], acc[bm][bn]);
    }
    // block (bm, bn) register e: tile row BR / WR wr + 32 bm + 8 (e / 4) + 4 hl + e % 4, column
    // m0 + BC / WC wc + 32 bn + r32
#pragma unroll
    for (int bn = 0; bn < NB; bn++) {
      const int col = m0 + BC / WC * wc + 32 * bn + r32;
#pragma unroll
      for (int bm = 0; bm < MB; bm++)
#pragma unroll
        for (int e = 0; e < 16; e++) {
          const int64_t row = (int64_t)rt * BR + BR / WR * wr + 32 * bm + 8 * (e >> 2) + 4 * hl + (e & 3);
          if (row < R && col < M) y[row * M + col] = acc[bm][bn][e];
        }
    }
    __syncthreads();  // every wave has read the X planes before the next tile's are written
  }
}

// The outer-product-mean operands from the MSA in one kernel: x = mask[s][n] (LN(m[s][n]) . W_ab[ch]) for the 64
// channels ch (a = 0..31, b = 32..63), fp32-accurate as above, written as the three bf16 parts in the chunk layout
// of bzpf_opm_split (chunk (g, n, p, h) at byte ((g N + n) 6 + 2 p + h) 1024: 32 channel rows of 16 MSA rows, zeros
// past S). Replaces bzpf_layernorm + bzpf_linear (a | b) + bzpf_opm_split. A tile is stage g (MSA rows 16 g .. + 15)
// of tokens 8 nb .. + 7: tile row 16 tl + k is (s = 16 g + k, n = 8 nb + tl). Wave w computes tile rows 32 w .. + 31
// (tokens 2 w, 2 w + 1) against the 64 channels (blocks h = a, b), so its accumulators hold whole chunk rows.
__global__ __launch_bounds__(256, 2) void opm_ln_split_k(const float* __restrict__ m, const float* __restrict__ lnw,
                                                         const float* __restrict__ lnb, float eps,
                                                         const float* __restrict__ w, const float* __restrict__ mask,
                                                         __bf16* __restrict__ planes, int S, int N, int nnb,
                                                         int ntiles) {
  __shared__ __attribute__((aligned(16))) char Ws[3 * 64 * LNP_ROWB];      // 24 KB: W_ab's three planes
  __shared__ __attribute__((aligned(16))) char Xs[3 * LNP_BR * LNP_ROWB];  // 48 KB: the tile's LN(m) planes
  __shared__ float Ms[LNP_BR];                                             // the tile rows' mask values
  const int t = threadIdx.x, wave = t >> 6, l = t & 63, r32 = l & 31, hl = l >> 5;
  // W_ab split once: f4 item e = t + 256 v is row e / 16, k = 4 (e % 16) .. + 3
#pragma unroll
  for (int v = 0; v < 4; v++) {
    const int e = t + 256 * v, row = e >> 4, kq = e & 15;
    const f4 a = *reinterpret_cast<const f4*>(w + row * LNP_K + 4 * kq);
    const Pair3 q01 = split3_pair(a[0], a[1]), q23 = split3_pair(a[2], a[3]);
#pragma unroll
    for (int p = 0; p < 3; p++)
      *reinterpret_cast<uint2*>(Ws + p * 64 * LNP_ROWB + lnp_off(row, kq >> 1) + 8 * (kq & 1)) =
          uint2{q01.p[p], q23.p[p]};
  }
  // m rows: pass v takes tile row t / 16 + 16 v, lane c = t % 16 channels 4 c .. + 3 (rows past S or N read a valid
  // row; past S their mask is taken as 0, past N their outputs are not stored)
  const int xc = t & 15, xr = t >> 4;
  const f4 gw = *reinterpret_cast<const f4*>(lnw + 4 * xc), gb = *reinterpret_cast<const f4*>(lnb + 4 * xc);
  f4 xv[8];
  float mv[8];
  auto xload = [&](int tile) {
    const int g = tile / nnb, nb = tile % nnb;
#pragma unroll
    for (int v = 0; v < 8; v++) {
      const int row = xr + 16 * v, s = 16 * g + (row & 15), n = min(8 * nb + (row >> 4), N - 1);
      const int64_t src = (int64_t)min(s, S - 1) * N + n;
      xv[v] = *reinterpret_cast<const f4*>(m + src * LNP_K + 4 * xc);
      const float mk = mask[src];
      mv[v] = s < S ? mk : 0.0f;
    }
  };
  auto xstage = [&]() {
#pragma unroll
    for (int v = 0; v < 8; v++) {
      const f4 a = xv[v];
      float s = 0.f;
      s += a[0] + a[1] + a[2] + a[3];
      const float mean = group_sum<16>(s) * (1.0f / LNP_K);
      float ss = 0.f;
      const f4 d = a - mean;
      ss += d[0] * d[0] + d[1] * d[1] + d[2] * d[2] + d[3] * d[3];
      const float rstd = 1.0f / sqrtf(group_sum<16>(ss) * (1.0f / LNP_K) + eps);
      f4 o = (a - mean) * rstd;
      o *= gw;
      o += gb;
      const Pair3 q01 = split3_pair(o[0], o[1]), q23 = split3_pair(o[2], o[3]);
      const int row = xr + 16 * v;
#pragma unroll
      for (int p = 0; p < 3; p++)
        *reinterpret_cast<uint2*>(Xs + p * LNP_BR * LNP_ROWB + lnp_off(row, xc >> 1) + 8 * (xc & 1)) =
            uint2{q01.p[p], q23.p[p]};
      if (xc == 0) Ms[row] = mv[v];
    }
  };
  int tile = (int)blockIdx.x;
  if (tile < ntiles) xload(tile);
  for (; tile < ntiles; tile += (int)gridDim.x) {  // workgroup-uniform
    xstage();
    __syncthreads();  // the X planes, the masks (and, the first time, the W planes) are complete
    if (tile + (int)gridDim.x < ntiles) xload(tile + (int)gridDim.x);
    f16x acc[2];
#pragma unroll
    for (int h = 0; h < 2; h++)
#pragma unroll
      for (int e = 0; e < 16; e++) acc[h][e] = 0.0f;
#pragma unroll
    for (int kk = 0; kk < LNP_K / 16; kk++) {
      bf16x8 fa[3], fb[2][3];
#pragma unroll
      for (int p = 0; p < 3; p++)
        fa[p] = *reinterpret_cast<const bf16x8*>(Xs + p * LNP_BR * LNP_ROWB + lnp_off(32 * wave + r32, 2 * kk + hl));
#pragma unroll
      for (int h = 0; h < 2; h++)
#pragma unroll
        for (int p = 0; p < 3; p++)
          fb[h][p] = *reinterpret_cast<const bf16x8*>(Ws + p * 64 * LNP_ROWB + lnp_off(32 * h + r32, 2 * kk + hl));
#pragma unroll
      for (int h = 0; h < 2; h++) acc[h] = mfma_parts6(fa, fb[h], acc[h]);
    }
    // register e of block h: tile row 32 wave + 8 (e / 4) + 4 hl + e % 4 = token 2 wave + e / 8, MSA row
    // k = 8 ((e / 4) % 2) + 4 hl + e % 4 of the stage; channel 32 h + r32. Registers e, e + 1 (e even) are MSA rows
    // k, k + 1: one dword per part.
    const int g = tile / nnb, nb = tile % nnb;
#pragma unroll
    for (int tk = 0; tk < 2; tk++) {
      const int n = 8 * nb + 2 * wave + tk;
      if (n >= N) continue;  // wave-uniform
      char* cbase = reinterpret_cast<char*>(planes) + ((int64_t)g * N + n) * 6144 + r32 * 32;
#pragma unroll
      for (int j = 0; j < 2; j++) {
        const int e0 = 8 * tk + 4 * j, k = 8 * j + 4 * hl;
        const int trow = 32 * wave + 16 * tk + k;
#pragma unroll
        for (int h = 0; h < 2; h++) {
          const Pair3 q01 = split3_pair(acc[h][e0] * Ms[trow], acc[h][e0 + 1] * Ms[trow + 1]);
          const Pair3 q23 = split3_pair(acc[h][e0 + 2] * Ms[trow + 2], acc[h][e0 + 3] * Ms[trow + 3]);
#pragma unroll
          for (int p = 0; p < 3; p++)
            *reinterpret_cast<uint2*>(cbase + (2 * p + h) * 1024 + 2 * k) = uint2{q01.p[p], q23.p[p]};
        }
      }
    }
    __syncthreads();  // every wave has read the X planes and masks before the next tile's are written
  }
}

// The 64-channel Transition in fp16 as one persistent kernel, in place: x += fc3(silu(xn fc1^T) * (xn fc2^T)) with
// xn = fp16(LN(x; ln_w, ln_b, eps)) for fp32 x [R, 64], w12 fp16 [2H, 64] = [fc1; fc2], w3 fp16 [64, H]
// (boltz_mlx/layers/transition.py:27-92 at 64 channels: the MSA track's transition and the template stack's; the
// fp16 overflow margin is folded into the weights by the caller). A wave takes 32 rows; everything runs transposed,
// so that a lane keeps one row throughout: h^T = W1 xn^T (the hidden units in a block's registers, the row in its
// lane), a = silu(h1) h2 rounded to fp16 is then already the B fragment of out^T = W3 a^T, and out^T's registers are
// the row's channels, added to the x values the lane loaded for the LayerNorm. The K order of each product is
// permuted within groups of 16 (lane half hl takes k = 4 hl .. + 3 and 8 + 4 hl .. + 3), which is where the
// accumulator layout puts a lane's values; the weights are staged in LDS with the same permutation, so each
// fragment is one 16-byte read. All weights stay in LDS (384 H bytes, H a multiple of 64); 8 waves, one workgroup
// per CU.
constexpr int TR64_MAXH = 384;

// position of k within its 16-group in the permuted order: j = 8 hl + 4 q + i holds k = 4 hl + i + 8 q
__device__ __forceinline__ int tr64_perm(int j) { return 4 * ((j >> 3) & 1) + (j & 3) + 8 * ((j >> 2) & 1); }

__global__ __launch_bounds__(512, 1) void transition64_f16_k(float* __restrict__ x, const float* __restrict__ lnw,
                                                             const float* __restrict__ lnb, float eps,
                                                             const half_t* __restrict__ w12,
                                                             const half_t* __restrict__ w3, int64_t R, int H,
                                                             int ntiles) {
  extern __shared__ __attribute__((aligned(16))) char tr64_lds[];
  half_t* W12s = reinterpret_cast<half_t*>(tr64_lds);  // [2H][64] permuted, 16-byte chunks swizzled by row % 8
  half_t* W3s = W12s + 2 * H * 64;                      // [64][H] permuted, chunks swizzled by row % 8
  const int t = threadIdx.x, wave = t >> 6, l = t & 63, r32 = l & 31, hl = l >> 5;
  // stage the weights: element (row, k) goes to k's permuted position, 16-byte chunk c of a row to c ^ (row % 8)
  for (int e = t; e < 2 * H * 64; e += 512) {
    const int row = e >> 6, j = e & 63, g = j & ~15;
    const int k = g + tr64_perm(j & 15);
    W12s[row * 64 + 8 * (((j >> 3) ^ (row & 7)) & 7) + (j & 7)] = w12[row * 64 + k];
  }
  for (int e = t; e < 64 * H; e += 512) {
    const int row = e / H, j = e % H, g = j & ~15;
    const int k = g + tr64_perm(j & 15);
    const int c = j >> 3, cs = (c & ~7) | ((c ^ row) & 7);
    W3s[row * H + 8 * cs + (j & 7)] = w3[row * H + k];
  }
  // lane (r32, hl) of wave w: row 32 w + r32 of the tile, channels 8 q + 4 hl .. + 3 for q = 0..7
  const f4* gw = reinterpret_cast<const f4*>(lnw);
  const f4* gb = reinterpret_cast<const f4*>(lnb);
  f4 xv[8], xn_next[8];
  auto xload = [&](f4 (&dst)[8], int tile) {
    const int64_t r = min((int64_t)tile * 256 + 32 * wave + r32, R - 1);
#pragma unroll
    for (int q = 0; q < 8; q++) dst[q] = *reinterpret_cast<const f4*>(x + r * 64 + 8 * q + 4 * hl);
  };
  int tile = (int)blockIdx.x;
  if (tile < ntiles) xload(xv, tile);
  __syncthreads();  // the weights are staged
  for (; tile < ntiles; tile += (int)gridDim.x) {  // workgroup-uniform
    if (tile + (int)gridDim.x < ntiles) xload(xn_next, tile + (int)gridDim.x);
    // LayerNorm over the row's 64 channels (the lane pair hl = 0, 1), then the fp16 B fragments of xn^T
    float s = 0.f;
#pragma unroll
    for (int q = 0; q < 8; q++) s += xv[q][0] + xv[q][1] + xv[q][2] + xv[q][3];
    s += __shfl_xor(s, 32, 64);
    const float mean = s * (1.0f / 64);
    float ss = 0.f;
#pragma unroll
    for (int q = 0; q < 8; q++) {
      const f4 d = xv[q] - mean;
      ss += d[0] * d[0] + d[1] * d[1] + d[2] * d[2] + d[3] * d[3];
    }
    ss += __shfl_xor(ss, 32, 64);
    const float rstd = 1.0f / sqrtf(ss * (1.0f / 64) + eps);
    half8 xb[4];
#pragma unroll
    for (int q = 0; q < 8; q++) {
      f4 o = (xv[q] - mean) * rstd;
      o *= gw[2 * q + hl];
      o += gb[2 * q + hl];
#pragma unroll
      for (int i = 0; i < 4; i++) xb[q >> 1][4 * (q & 1) + i] = (half_t)o[i];
    }
    f16x out[2];
#pragma unroll
    for (int b = 0; b < 2; b++)
#pragma unroll
      for (int e = 0; e < 16; e++) out[b][e] = 0.0f;
    for (int c = 0; c < H / 32; c++) {
      f16x h1, h2;
#pragma unroll
      for (int e = 0; e < 16; e++) h1[e] = h2[e] = 0.0f;
      const int u = 32 * c + r32;  // the A rows (hidden units) of this lane
#pragma unroll
      for (int kk = 0; kk < 4; kk++) {
        const int ch = ((2 * kk + hl) ^ (u & 7)) & 7;
        const half8 a1 = *reinterpret_cast<const half8*>(W12s + u * 64 + 8 * ch);
        const half8 a2 = *reinterpret_cast<const half8*>(W12s + (H + u) * 64 + 8 * ch);
        h1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a1, xb[kk], h1, 0, 0, 0);
        h2 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a2, xb[kk], h2, 0, 0, 0);
      }
      // register e: hidden unit 32 c + 8 (e / 4) + 4 hl + e % 4 of this lane's row; k-step kk2 of fc3 takes
      // e = 8 kk2 .. + 7 (units 32 c + 16 kk2 + the permuted group)
      half8 ab[2];
#pragma unroll
      for (int e = 0; e < 16; e++) ab[e >> 3][e & 7] = (half_t)(siluf_(h1[e]) * h2[e]);
#pragma unroll
      for (int kk2 = 0; kk2 < 2; kk2++) {
        const int cc = (32 * c + 16 * kk2 + 8 * hl) >> 3;
#pragma unroll
        for (int b = 0; b < 2; b++) {
          const int d = 32 * b + r32;
          const int cs = (cc & ~7) | ((cc ^ d) & 7);
          const half8 a3 = *reinterpret_cast<const half8*>(W3s + d * H + 8 * cs);
          out[b] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a3, ab[kk2], out[b], 0, 0, 0);
        }
      }
    }
    // out[b] register e: channel 32 b + 8 (e / 4) + 4 hl + e % 4 = 8 q + 4 hl + i with q = 4 b + e / 4
    const int64_t r = (int64_t)tile * 256 + 32 * wave + r32;
    if (r < R) {
#pragma unroll
      for (int q = 0; q < 8; q++) {
        const f4 o = f4{out[q >> 2][4 * (q & 3)], out[q >> 2][4 * (q & 3) + 1], out[q >> 2][4 * (q & 3) + 2],
                        out[q >> 2][4 * (q & 3) + 3]};
        *reinterpret_cast<f4*>(x + r * 64 + 8 * q + 4 * hl) = xv[q] + o;
      }
    }
#pragma unroll
    for (int q = 0; q < 8; q++) xv[q] = xn_next[q];
  }
}

}  // namespace

hipError_t launch_transition64_f16(float* x, const float* lnw, const float* lnb, float eps, const void* w12,
                                   const void* w3, int64_t R, int H, hipStream_t st) {
  const auto al = [](const void* p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0; };
  if (R < 1 || H < 64 || H % 64 || H > TR64_MAXH || !lnw || !lnb || !al(x, 16) || !al(lnw, 16) || !al(lnb, 16) ||
      (R + 255) / 256 > INT32_MAX)
    return hipErrorInvalidValue;
  const size_t lds = (size_t)384 * H;
  static bool attr_set[kMaxDevices];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
  if (!attr_set[dev]) {
    const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(transition64_f16_k),
                                             hipFuncAttributeMaxDynamicSharedMemorySize, 384 * TR64_MAXH);
    if (e != hipSuccess) return e;
    attr_set[dev] = true;
  }
  int cus = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus < 1)
    return hipErrorInvalidDevice;
  const int ntiles = (int)((R + 255) / 256);
  transition64_f16_k<<<min(ntiles, cus), 512, lds, st>>>(x, lnw, lnb, eps, static_cast<const half_t*>(w12),
                                                         static_cast<const half_t*>(w3), R, H, ntiles);
  return hipGetLastError();
}

hipError_t launch_opm_ln_split(const float* m, const float* lnw, const float* lnb, float eps, const float* w_ab,
                               const float* mask, void* planes, int S, int N, hipStream_t st) {
  const auto al = [](const void* p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0; };
  if (S < 1 || N < 1 || !lnw || !lnb || !al(m, 16) || !al(w_ab, 16) || !al(lnw, 16) || !al(lnb, 16) ||
      !al(planes, 16) || (int64_t)N * 6144 > INT32_MAX)
    return hipErrorInvalidValue;
  const int64_t G = (S + 15) / 16, nnb = (N + 7) / 8;
  if (G * nnb > INT32_MAX) return hipErrorInvalidValue;
  static int cache[kMaxDevices];
  const int resident = resident_grid(opm_ln_split_k, 256, cache);
  if (resident <= 0) return hipErrorInvalidDevice;
  const int ntiles = (int)(G * nnb);
  opm_ln_split_k<<<min(ntiles, resident), 256, 0, st>>>(m, lnw, lnb, eps, w_ab, mask, static_cast<__bf16*>(planes), S,
                                                       N, (int)nnb, ntiles);
  return hipGetLastError();
}

template <int BR, int BC, int WR, int WC>
static hipError_t ln_linear_x3_t(const float* x, const float* lnw, const float* lnb, float eps, const float* w, float* y,
                                 int64_t R, int M, hipStream_t st) {
  static int cache[kMaxDevices];
  const int resident = resident_grid(ln_linear_x3_k<BR, BC, WR, WC>, 64 * WR * WC, cache);
  if (resident <= 0) return hipErrorInvalidDevice;
  const int ncb = M / BC, nrt = (int)((R + BR - 1) / BR);
  // whole groups of ncb workgroups (one per column block), no more row-tile slots than row tiles
  const int per_cb = max(1, min(nrt, resident / ncb));
  ln_linear_x3_k<BR, BC, WR, WC><<<ncb * per_cb, 64 * WR * WC, 0, st>>>(x, lnw, lnb, eps, w, y, R, M, ncb, nrt);
  return hipGetLastError();
}

hipError_t launch_ln_linear_x3(const float* x, const float* lnw, const float* lnb, float eps, const float* w, float* y,
                               int64_t R, int K, int M, hipStream_t st) {
  const auto al = [](const void* p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0; };
  if (R < 1 || K != LNP_K || M < LNP_BC || M % LNP_BC || !lnw || !lnb || !al(x, 16) || !al(w, 16) || !al(lnw, 16) ||
      !al(lnb, 16) || (R + LNP_BR - 1) / LNP_BR > INT32_MAX)
    return hipErrorInvalidValue;
  return ln_linear_x3_t<128, 256, 2, 4>(x, lnw, lnb, eps, w, y, R, M, st);
}

}  // namespace bzpf
