// The row-GEMM kernels of the pair track, all on the transposed row-tile scheme of bzpf_rowgemm.h (Y^T = W X^T with
// X rows in registers and W streamed through LDS in 64-channel chunks):
//   trimul_proj      : ab[c][i][k] = (xn W_p[c]) * sigmoid(xn W_g[c]) * mask * scale at (i, k) (incoming: (k, i))
//                      (boltz_mlx/layers/triangular_mult.py:67-88, 143-170; kernels_nax2.py:202-304);
//   trimul_tail      : z (+)= p_out(LN_out(o)) * sigmoid(g_out(xn)), then the next LayerNorm
//                      (triangular_mult.py:98-118; kernels_nax3.py:200-268, 1061-1206);
//   triattn_proj     : q|k|v|g planes, V^T rows and the triangle bias (attention.py:49-69, 100-104);
//   linear_resid_ln  : z (+)= x W_o^T at the (transposed) position, then the next LayerNorm (kernels_nax3.py:176-198);
//   transition       : z (+)= fc3(silu(fc1 xn) * fc2 xn), then the next LayerNorm (transition.py:27-54, 148-154;
//                      kernels_nax2.py:54-190, kernels_nax3.py:713-827).
// Tiles are 64 * RB rows (positions) per workgroup of 4 waves, RB = 2 row blocks per wave for fp16 and 1 for fp32.
#include "bzpf_common.h"
#include "bzpf_kernels.h"
#include "bzpf_rowgemm.h"

namespace bzpf {

namespace {

constexpr int D = 128;

template <typename T> constexpr int ldw_of() { return D + Pad<T>::v; }

// ---------------------------------------------------------------- triangle multiplication projection
// Persistent, one 512-thread workgroup per CU (8 waves, up to 256 VGPRs each). The launch covers output channels
// [c_lo, c_lo + PCH): the projection rows c_lo.. and gate rows 2D + c_lo.. of w (PCH = 256 in fp16: all of them;
// 128 in fp32, two launches) are staged in LDS once; each wave then streams tiles of HV TW positions
// (i, k0 .. k0 + HV TW) over the padded rows of length ld as HV halves of TW, computing (ROWS orientation) one
// 16-byte run per channel and half: with HV = 2 a whole 128-byte line of ab[c][i][k] (fp16) per channel row and
// tile, written by one wave with two adjacent stores (incoming: xn read at (k, i)). The next tile's rows and mask
// values are loaded while the current tile computes (8 waves with the prefetch measured 3-4% faster than 12
// without). HV = 1 (half tiles) is taken when it balances the last round of tiles better: at N = 400 (2,800 full
// tiles on 2,048 waves) 0.041-0.045 against 0.050 ms; at N = 1000 full tiles are faster (0.23 against 0.26 ms).
template <typename T> constexpr int proj_ch() { return sizeof(T) == 2 ? 256 : 128; }
constexpr int PROJ_WAVES = 8;

template <typename T, int HV>
__global__ __launch_bounds__(64 * PROJ_WAVES) void trimul_proj_k(const T* __restrict__ xn, const T* __restrict__ w,
                                                                 const float* __restrict__ mask, float scale,
                                                                 int incoming, T* __restrict__ ab, int64_t N,
                                                                 int64_t ld, int c_lo) {
  using RT = RunTile<T>;
  constexpr int RB = RT::RB, TW = RT::TW, STEPS = RG<T>::STEPS, LDW = ldw_of<T>(), PCH = proj_ch<T>();
  __shared__ LDS_ALIGN T Ws[2 * PCH * LDW];  // rows [0, PCH): projections, [PCH, 2 PCH): gates
  lds_rows<T>(Ws, LDW, 2 * PCH, D,
              [&](int r) { return w + (int64_t)(r < PCH ? c_lo + r : 2 * D + c_lo + r - PCH) * D; });
  __syncthreads();
  const int l = threadIdx.x & 63, g = l >> 4, r = l & 15;
  const int tpr = (int)(ld / (HV * TW)), ntiles = (int)N * tpr, stride = gridDim.x * PROJ_WAVES;
  int t = grid_wave(PROJ_WAVES);
  if (t >= ntiles) return;

  typedef typename RG<T>::frag Frag;
  Frag x[HV][RB][STEPS];
  // mask values of the rows this lane loads, raw (at the clamped position): scaled, and zeroed past N (padding columns
  // are written as 0), where they are used. Any arithmetic on them at the load would wait for the prefetch there.
  float mk[HV][RB];
  const auto load = [&](int tt, Frag (&xx)[HV][RB][STEPS], float (&mm)[HV][RB]) {
    const int i = tt / tpr, k0 = (tt - i * tpr) * HV * TW;
#pragma unroll
    for (int hh = 0; hh < HV; hh++)
#pragma unroll
      for (int rb = 0; rb < RB; rb++) {
        const int64_t k = k0 + hh * TW + RT::pos(rb, r), kc = k < N ? k : N - 1;
        const int64_t src = incoming ? kc * N + i : (int64_t)i * N + kc;
        RG<T>::load_row(xx[hh][rb], xn + src * D, g);
        mm[hh][rb] = mask[src];
      }
  };
  load(t, x, mk);
  for (; t < ntiles; t += stride) {
    Frag xnx[HV][RB][STEPS];
    float mkn[HV][RB];
    load(min(t + stride, ntiles - 1), xnx, mkn);
    const int i = t / tpr, k0 = (t - i * tpr) * HV * TW;
    float mo[HV][RB][4];  // mask of this lane's output positions RUN g + 4 rb + e of each half, from lane 4 g + e
#pragma unroll
    for (int hh = 0; hh < HV; hh++)
#pragma unroll
      for (int rb = 0; rb < RB; rb++) {
        const float mv = k0 + hh * TW + RT::pos(rb, r) < N ? mk[hh][rb] * scale : 0.0f;
#pragma unroll
        for (int e = 0; e < 4; e++) mo[hh][rb][e] = __shfl(mv, 4 * g + e);
      }
    T* dst = ab + ((int64_t)(c_lo + r) * N + i) * ld + k0 + RT::RUN * g;
    for (int cb = 0; cb < PCH / 16; cb++) {
#pragma unroll
      for (int hh = 0; hh < HV; hh++) {
        f4 pa[RB][1], ga[RB][1];
        zero_acc(pa);
        zero_acc(ga);
        mma_rows<T, RB, 1, true>(pa, x[hh], Ws + 16 * cb * LDW, LDW);
        mma_rows<T, RB, 1, true>(ga, x[hh], Ws + (PCH + 16 * cb) * LDW, LDW);
        float v[RT::RUN];
#pragma unroll
        for (int rb = 0; rb < RB; rb++)
#pragma unroll
          for (int e = 0; e < 4; e++) v[4 * rb + e] = pa[rb][0][e] * sigmoidf_(ga[rb][0][e]) * mo[hh][rb][e];
        st_run_cached(dst + (int64_t)16 * cb * N * ld + hh * TW, v);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int hh = 0; hh < HV; hh++)
#pragma unroll
      for (int rb = 0; rb < RB; rb++) {
        mk[hh][rb] = mkn[hh][rb];
#pragma unroll
        for (int s2 = 0; s2 < STEPS; s2++) x[hh][rb][s2] = xnx[hh][rb][s2];
      }
  }
}

// ---------------------------------------------------------------- triangle multiplication tail
// grid: N * tiles_per_row over the padded rows (positions (i, j0 .. j0+TM)).
template <typename T>
__global__ __launch_bounds__(256) void trimul_tail_k(const T* __restrict__ o, const float* __restrict__ now,
                                                     const float* __restrict__ nob, float eps_out,
                                                     const T* __restrict__ w_po, const T* __restrict__ xn,
                                                     const T* __restrict__ w_go, float* __restrict__ z, int accumulate,
                                                     const float* __restrict__ lnw, const float* __restrict__ lnb,
                                                     float eps_next, T* __restrict__ xn_next, int64_t N, int64_t ld) {
  constexpr int RB = RowBlocks<T>::v, TM = 64 * RB, STEPS = RG<T>::STEPS, LDW = ldw_of<T>();
  __shared__ LDS_ALIGN T Ts[TM * LDW];  // o tile transposed to [position][channel], then LN_out of it
  __shared__ LDS_ALIGN T Ws[64 * LDW];
  const int64_t tpr = (ld + TM - 1) / TM;
  const int64_t i = blockIdx.x / tpr;
  const int64_t j0 = (blockIdx.x - i * tpr) * TM;
  const int wave = threadIdx.x >> 6, l = threadIdx.x & 63, g = l >> 4;

  // o tile: each channel row holds contiguous positions (columns past ld are not read)
  {
    constexpr int VE = Vec16<T>::n;
    for (int e = threadIdx.x; e < D * (TM / VE); e += 256) {
      const int c = e / (TM / VE), r = (e - c * (TM / VE)) * VE;
      if (j0 + r >= ld) continue;
      U128 v = *reinterpret_cast<const U128*>(o + ((int64_t)c * N + i) * ld + j0 + r);
      const T* vv = reinterpret_cast<const T*>(&v);
#pragma unroll
      for (int u = 0; u < VE; u++) Ts[(r + u) * LDW + c] = vv[u];
    }
  }
  __syncthreads();
  // LN_out over the 128 channels of each position (4 threads per row, two-pass fp32 statistics)
  for (int r = threadIdx.x >> 2; r < TM; r += 64) {
    const int q = threadIdx.x & 3;
    T* tr = Ts + r * LDW + q * 32;
    float v[32];
    float s = 0.f;
#pragma unroll
    for (int c = 0; c < 32; c++) { v[c] = to_f(tr[c]); s += v[c]; }
    const float mean = group_sum<4>(s) * (1.0f / D);
    float ss = 0.f;
#pragma unroll
    for (int c = 0; c < 32; c++) { const float d = v[c] - mean; ss += d * d; }
    const float rstd = 1.0f / sqrtf(group_sum<4>(ss) * (1.0f / D) + eps_out);
#pragma unroll
    for (int c = 0; c < 32; c++) tr[c] = from_f<T>((v[c] - mean) * rstd * now[q * 32 + c] + nob[q * 32 + c]);
  }
  int64_t jpos[RB];
  typename RG<T>::frag x[RB][STEPS];
#pragma unroll
  for (int rb = 0; rb < RB; rb++) {
    jpos[rb] = j0 + wave * 16 * RB + 16 * rb + (l & 15);
    const int64_t jc = jpos[rb] < N ? jpos[rb] : N - 1;
    RG<T>::load_row(x[rb], xn + (i * N + jc) * D, g);
  }
  // gates sigmoid(xn W_go^T), two 64-channel chunks
  f4 gate[RB][8];
#pragma unroll
  for (int cc = 0; cc < 2; cc++) {
    __syncthreads();
    lds_rows<T>(Ws, LDW, 64, D, [&](int r) { return w_go + (int64_t)(64 * cc + r) * D; });
    __syncthreads();
    f4 acc[RB][4];
    zero_acc(acc);
    mma_rows<T, RB, 4>(acc, x, Ws, LDW);
#pragma unroll
    for (int rb = 0; rb < RB; rb++)
#pragma unroll
      for (int cb = 0; cb < 4; cb++)
#pragma unroll
        for (int e = 0; e < 4; e++) gate[rb][4 * cc + cb][e] = sigmoidf_(acc[rb][cb][e]);
  }
  // LN_out rows as the B operand, p_out chunks
#pragma unroll
  for (int rb = 0; rb < RB; rb++) RG<T>::load_row(x[rb], Ts + (wave * 16 * RB + 16 * rb + (l & 15)) * LDW, g);
  f4 y[RB][8];
#pragma unroll
  for (int cc = 0; cc < 2; cc++) {
    __syncthreads();
    lds_rows<T>(Ws, LDW, 64, D, [&](int r) { return w_po + (int64_t)(64 * cc + r) * D; });
    __syncthreads();
    f4 acc[RB][4];
    zero_acc(acc);
    mma_rows<T, RB, 4>(acc, x, Ws, LDW);
#pragma unroll
    for (int rb = 0; rb < RB; rb++)
#pragma unroll
      for (int cb = 0; cb < 4; cb++) y[rb][4 * cc + cb] = acc[rb][cb] * gate[rb][4 * cc + cb];
  }
  resid_ln_rows<T, RB>(y, [&](int rb) -> int64_t { return jpos[rb] < N ? i * N + jpos[rb] : -1; }, z, accumulate, lnw,
                       lnb, eps_next, xn_next);
}

// fp16 tail, persistent: one 768-thread workgroup per CU (12 waves, 3 per SIMD) with g_out and p_out resident in LDS.
// LN_out's affine part is folded into p_out when it is staged (columns scaled by gamma, bias W_po . beta), so the
// kernel only normalises. Each wave streams tiles of 16 positions (i, j0 .. j0 + 15): its lanes load 4-channel x
// 8-position blocks of the channel-major o (lane l: channels 4 (l / 2) .. + 3, positions 8 (l % 2) .. + 7), write
// them as [position][channel] rows of a wave-private LDS tile (two byte permutes per position) and read the usual
// row fragments back, with no barrier (a wave's LDS accesses complete in order). The next tile's o block and gate
// inputs are loaded while the current tile computes; its residual rows are issued at the start of the tile. The
// gates are computed first and held as fp16 (sigmoid values in (0, 1)), which keeps the tile within 168 VGPRs.
// One 128-byte line of an o channel row holds 64 positions, i.e. four tiles. Tiles per row are a multiple of four
// (tiles past N store nothing), so the workgroup's 12 consecutive tiles hold whole lines, and one barrier per round
// keeps its waves in step: the four loads of a line reach L2 together and it is read from HBM once. Without the
// barrier the waves drift apart by more than the L2 residency of a line and o is read about 2.3 times.
constexpr int TAIL_WAVES = 12;
__host__ __device__ constexpr int64_t tail_tiles_per_row(int64_t N) { return (N + 63) / 64 * 4; }

__global__ __launch_bounds__(64 * TAIL_WAVES) void trimul_tail_f16_k(
    const half_t* __restrict__ o, const float* __restrict__ now, const float* __restrict__ nob, float eps_out,
    const half_t* __restrict__ w_po, const half_t* __restrict__ xn, const half_t* __restrict__ w_go,
    float* __restrict__ z, int accumulate, const float* __restrict__ lnw, const float* __restrict__ lnb,
    float eps_next, half_t* __restrict__ xn_next, int64_t N, int64_t ld) {
  using T = half_t;
  constexpr int STEPS = RG<T>::STEPS, LDW = ldw_of<T>(), LDT = D + Pad<T>::v;
  __shared__ LDS_ALIGN T Wg[D * LDW];
  __shared__ LDS_ALIGN T Wp[D * LDW];  // p_out with gamma_out folded into its columns
  __shared__ LDS_ALIGN float Bp[D];    // p_out . beta_out
  __shared__ LDS_ALIGN float Lw[D], Lb[D];  // the next LayerNorm (read per lane from LDS, not by hoisted pointers)
  __shared__ LDS_ALIGN T Ts[TAIL_WAVES][16 * LDT];
  lds_rows<T>(Wg, LDW, D, D, [&](int r) { return w_go + (int64_t)r * D; });
  for (int e = threadIdx.x; e < D * D / 8; e += blockDim.x) {
    const int r = e >> 4, c = (e & 15) * 8;
    const half8 wv = *reinterpret_cast<const half8*>(w_po + (int64_t)r * D + c);
    half8 sv;
#pragma unroll
    for (int u = 0; u < 8; u++) sv[u] = (half_t)((float)wv[u] * now[c + u]);
    *reinterpret_cast<half8*>(Wp + r * LDW + c) = sv;
  }
  if (lnw != nullptr && threadIdx.x < D) {
    Lw[threadIdx.x] = lnw[threadIdx.x];
    Lb[threadIdx.x] = lnb[threadIdx.x];
  }
  if (threadIdx.x < 4 * D) {  // 4 lanes per output channel, 32 inputs each
    const int c = threadIdx.x >> 2, q = threadIdx.x & 3;
    float acc = 0.f;
#pragma unroll
    for (int v = 0; v < 4; v++) {
      const half8 wv = *reinterpret_cast<const half8*>(w_po + (int64_t)c * D + 32 * q + 8 * v);
#pragma unroll
      for (int u = 0; u < 8; u++) acc += (float)wv[u] * nob[32 * q + 8 * v + u];
    }
    acc += __shfl_xor(acc, 1, 64);
    acc += __shfl_xor(acc, 2, 64);
    if (q == 0) Bp[c] = acc;
  }
  __syncthreads();

  const int l = threadIdx.x & 63, g = l >> 4, r = l & 15;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  T* ts = Ts[wave];
  const int tpr = (int)tail_tiles_per_row(N), ntiles = (int)N * tpr, stride = gridDim.x * TAIL_WAVES;
  // rounds are workgroup-uniform (the barrier below needs every wave in every round); a wave whose tile is past the
  // end of a round recomputes the last tile and stores nothing
  int tb = blockIdx.x * TAIL_WAVES;
  if (tb >= ntiles) return;  // whole workgroup
  int t = min(tb + wave, ntiles - 1);
  const int ocg = l >> 1, opc = l & 1;
  // o element offsets are 32-bit (the launcher checks D * N * ld < 2^31): channel rows of this lane, one apart
  const uint32_t ochan = (uint32_t)(4 * ocg) * (uint32_t)N * (uint32_t)ld, orow = (uint32_t)N * (uint32_t)ld;
  const auto load = [&](int tt, half8 (&ob)[4], typename RG<T>::frag (&xf)[1][STEPS]) {
    const int i = tt / tpr, j0 = (tt - i * tpr) * 16;
    const uint32_t oo = ochan + (uint32_t)i * (uint32_t)ld + (uint32_t)(j0 + 8 * opc);
#pragma unroll
    for (int u = 0; u < 4; u++) ob[u] = *reinterpret_cast<const half8*>(o + (oo + u * orow));
    const int64_t jc = j0 + r < N ? j0 + r : N - 1;
    RG<T>::load_row(xf[0], xn + ((int64_t)i * N + jc) * D, g);
  };
  half8 ob[4];
  typename RG<T>::frag xf[1][STEPS];
  load(t, ob, xf);
  for (; tb < ntiles; tb += stride) {
    const bool live = tb + wave < ntiles;
    t = live ? tb + wave : ntiles - 1;
    __syncthreads();
    const int i = t / tpr, j0 = (t - i * tpr) * 16;
    const int64_t zr = live && j0 + r < N ? (int64_t)i * N + j0 + r : -1;
    const auto zrow = [&](int) { return zr; };
    float* zt = opaque_ptr(z);
    half_t* xnt = opaque_ptr(xn_next);
    f4 zv[1][8];
    load_z_rows<1>(zv, zrow, zt, accumulate);
    // o block -> [position][channel] rows of the wave's tile
#pragma unroll
    for (int v = 0; v < 8; v++)
      *reinterpret_cast<half4*>(ts + (8 * opc + v) * LDT + 4 * ocg) = half4{ob[0][v], ob[1][v], ob[2][v], ob[3][v]};
    half8 obn[4];
    typename RG<T>::frag xfn[1][STEPS];
    load(min(t + stride, ntiles - 1), obn, xfn);
    // gates first (their inputs are free afterwards), kept as fp16
    half4 gate[8];
    {
      f4 ga[1][8];
      zero_acc(ga);
      mma_rows_grouped<T, 1, 8, 1>(ga, xf, Wg, LDW);
#pragma unroll
      for (int cb = 0; cb < 8; cb++)
        gate[cb] = half4{(half_t)sigmoidf_(ga[0][cb][0]), (half_t)sigmoidf_(ga[0][cb][1]),
                         (half_t)sigmoidf_(ga[0][cb][2]), (half_t)sigmoidf_(ga[0][cb][3])};
    }
    // LN_out of this lane's position (channels 32 g .. 32 g + 31 here, the rest in lanes l ^ 16, l ^ 32, l ^ 48)
    typename RG<T>::frag of[1][STEPS];
    RG<T>::load_row(of[0], ts + r * LDT, g);
    float sum = 0.f;
#pragma unroll
    for (int s2 = 0; s2 < STEPS; s2++)
#pragma unroll
      for (int u = 0; u < 8; u++) sum += (float)of[0][s2][u];
    const float mean = xgroups_sum(sum) * (1.0f / D);
    float ss = 0.f;
#pragma unroll
    for (int s2 = 0; s2 < STEPS; s2++)
#pragma unroll
      for (int u = 0; u < 8; u++) {
        const float d = (float)of[0][s2][u] - mean;
        ss += d * d;
      }
    const float rstd = 1.0f / sqrtf(xgroups_sum(ss) * (1.0f / D) + eps_out);
#pragma unroll
    for (int s2 = 0; s2 < STEPS; s2++)
#pragma unroll
      for (int u = 0; u < 8; u++) of[0][s2][u] = (half_t)(((float)of[0][s2][u] - mean) * rstd);
    f4 y[1][8];
    zero_acc(y);
    mma_rows_grouped<T, 1, 8, 1>(y, of, Wp, LDW);
#pragma unroll
    for (int cb = 0; cb < 8; cb++) {
      const f4 bp = *reinterpret_cast<const f4*>(Bp + 16 * cb + 4 * g);
#pragma unroll
      for (int e = 0; e < 4; e++) y[0][cb][e] = (y[0][cb][e] + bp[e]) * (float)gate[cb][e];
    }
    resid_ln_apply<T, 1>(y, zv, zrow, zt, lnw != nullptr ? Lw : nullptr, Lb, eps_next, xnt);
#pragma unroll
    for (int u = 0; u < 4; u++) ob[u] = obn[u];
#pragma unroll
    for (int s2 = 0; s2 < STEPS; s2++) xf[0][s2] = xfn[0][s2];
  }
}

// ---------------------------------------------------------------- triangle attention projection
// Persistent like trimul_proj. Rows of w: q [0, D), k [D, 2D), v [2D, 3D), g [3D, 4D), triangle bias [4D, 4D + H)
// (H * C = D). A launch stages the rows [r_lo, r_hi) of that list with the bias block padded to 16 zero rows
// (fp16: all 4D + 16 rows; fp32: [0, 2D) and [2D, 4D + 16) in two launches). Each wave streams tiles of TW positions
// (i, j0 .. j0 + TW) of the padded rows (length ldk), position (i, j) reading xn at (i, j) (trans: (j, i)):
//   q, k, g : transposed orientation; the staging permutes each 32-row group (LDS row 32 m + 16 c + rr holds channel
//             32 m + 8 (rr / 4) + 4 c + rr % 4), so the lane of group g holds channels 8 g .. 8 g + 7 of its position:
//             one 16-byte run of qkg[plane][i N + j][:] (q scaled by q_scale);
//   v       : ROWS orientation, 16-byte runs of keys of vt[h][i][d][:] (zeros past N);
//   bias    : ROWS orientation, runs of 4 keys of the fragment-ordered bias (scaled by b_scale, zeros past N).
template <typename T> constexpr int attn_rows() { return sizeof(T) == 2 ? 4 * D + 16 : 2 * D + 16; }

__device__ __forceinline__ void st8(half_t* p, const float (&v)[8]) { st_run(p, v); }
__device__ __forceinline__ void st8(float* p, const float (&v)[8]) {
  *reinterpret_cast<f4*>(p) = f4{v[0], v[1], v[2], v[3]};
  *reinterpret_cast<f4*>(p + 4) = f4{v[4], v[5], v[6], v[7]};
}

// 12 waves (3 per SIMD, up to 168 VGPRs): the two row sets (current and prefetched) plus the per-lane store addresses
// of the three output layouts do not fit the 128 VGPRs of 4 waves per SIMD.
constexpr int ATTN_PROJ_WAVES = 12;

template <typename T>
__global__ __launch_bounds__(64 * ATTN_PROJ_WAVES) void triattn_proj_k(const T* __restrict__ xn,
                                                                        const T* __restrict__ w, int trans,
                                                                        float q_scale, float b_scale,
                                                                        T* __restrict__ qkg, T* __restrict__ vt,
                                                                        T* __restrict__ tb, int64_t N, int64_t ldk,
                                                                        int H, int C, int r_lo, int r_hi) {
  using RT = RunTile<T>;
  constexpr int RB = RT::RB, TW = RT::TW, STEPS = RG<T>::STEPS, LDW = ldw_of<T>();
  __shared__ LDS_ALIGN T Ws[attn_rows<T>() * LDW];
  lds_rows<T>(Ws, LDW, r_hi - r_lo, D, [&](int lr) -> const T* {
    const int R = r_lo + lr;
    if (R >= 4 * D) return R - 4 * D < H ? w + (int64_t)R * D : nullptr;
    if (R >= 2 * D && R < 3 * D) return w + (int64_t)R * D;
    const int q = R & 31, rr = q & 15;
    return w + (int64_t)((R & ~31) + 8 * (rr >> 2) + 4 * (q >> 4) + (rr & 3)) * D;
  });
  __syncthreads();
  const int l = threadIdx.x & 63, g = l >> 4, r = l & 15;
  const int64_t NN = N * N;
  const int tpr = (int)(ldk / TW), ntiles = (int)N * tpr, stride = gridDim.x * ATTN_PROJ_WAVES;
  int t = grid_wave(ATTN_PROJ_WAVES);
  if (t >= ntiles) return;

  typename RG<T>::frag x[RB][STEPS];
  const auto load = [&](int tt, typename RG<T>::frag (&xx)[RB][STEPS]) {
    const int i = tt / tpr, j0 = (tt - i * tpr) * TW;
#pragma unroll
    for (int rb = 0; rb < RB; rb++) {
      const int64_t j = j0 + RT::pos(rb, r), jc = j < N ? j : N - 1;
      RG<T>::load_row(xx[rb], xn + (trans ? jc * N + i : (int64_t)i * N + jc) * D, g);
    }
  };
  load(t, x);
  for (; t < ntiles; t += stride) {
    const int i = t / tpr, j0 = (t - i * tpr) * TW;
    typename RG<T>::frag xnext[RB][STEPS];
    load(min(t + stride, ntiles - 1), xnext);
    // ROWS orientation: key j0 + RUN g + 4 rb + e is inside the row
    const auto valid = [&](int rb, int e) { return j0 + RT::RUN * g + 4 * rb + e < N ? 1.0f : 0.0f; };
    for (int m = 0; m < r_hi - r_lo; m += 32) {
      const int R = r_lo + m;
      const T* wb = Ws + m * LDW;
      if (R >= 4 * D) {  // triangle bias (16-row block, H valid rows)
        f4 acc[RB][1];
        zero_acc(acc);
        mma_rows<T, RB, 1, true>(acc, x, wb, LDW);
        if (r < H) {
#pragma unroll
          for (int rb = 0; rb < RB; rb++) {
            const f4 v = acc[rb][0] * b_scale;
            st4(tb + tb_offset(r, i, j0 + RT::RUN * g + 4 * rb, N, ldk),
                f4{v[0] * valid(rb, 0), v[1] * valid(rb, 1), v[2] * valid(rb, 2), v[3] * valid(rb, 3)});
          }
        }
      } else if (R >= 2 * D && R < 3 * D) {  // v
        f4 acc[RB][2];
        zero_acc(acc);
        mma_rows_grouped<T, RB, 2, 1, true>(acc, x, wb, LDW);
#pragma unroll
        for (int c = 0; c < 2; c++) {
          const int ch = R - 2 * D + 16 * c + r, h = ch / C, d = ch - h * C;
          float v[RT::RUN];
#pragma unroll
          for (int rb = 0; rb < RB; rb++)
#pragma unroll
            for (int e = 0; e < 4; e++) v[4 * rb + e] = acc[rb][c][e] * valid(rb, e);
          st_run(vt + (((int64_t)h * N + i) * C + d) * ldk + j0 + RT::RUN * g, v);
        }
      } else {  // q, k, g
        f4 acc[RB][2];
        zero_acc(acc);
        mma_rows_grouped<T, RB, 2, 1, false>(acc, x, wb, LDW);
        const int P = R / D, within = R - P * D + 8 * g, h = within / C, d = within - h * C;
        const int64_t plane = (int64_t)(P == 3 ? 2 : P) * H + h;
        const float sc = P == 0 ? q_scale : 1.0f;
#pragma unroll
        for (int rb = 0; rb < RB; rb++) {
          const int64_t j = j0 + RT::pos(rb, r);
          if (j >= N) continue;
          const float v[8] = {acc[rb][0][0] * sc, acc[rb][0][1] * sc, acc[rb][0][2] * sc, acc[rb][0][3] * sc,
                              acc[rb][1][0] * sc, acc[rb][1][1] * sc, acc[rb][1][2] * sc, acc[rb][1][3] * sc};
          st8(qkg + (plane * NN + (int64_t)i * N + j) * C + d, v);
        }
      }
      __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int rb = 0; rb < RB; rb++)
#pragma unroll
      for (int s = 0; s < STEPS; s++) x[rb][s] = xnext[rb][s];
  }
}

// ---------------------------------------------------------------- linear_o + residual + next LayerNorm
// Persistent: W (128 x 128) is staged in LDS once per workgroup; each wave then streams 16-row tiles with no
// barriers. The rows and residual rows of the wave's next tile are loaded a whole tile ahead (one HBM round trip is
// longer than the compute of the waves sharing a SIMD). On a wave's last tile the clamped "next" tile may be another
// wave's; those loads are never used.
template <typename T>
__global__ __launch_bounds__(256, sizeof(T) == 2 ? 3 : 2) void linear_resid_ln_k(const T* __restrict__ x_in,
                                                                                const T* __restrict__ w, int trans,
                                                                                float* __restrict__ z, int accumulate,
                                                                                const float* __restrict__ lnw,
                                                                                const float* __restrict__ lnb,
                                                                                float eps, T* __restrict__ xn_next,
                                                                                int64_t N) {
  constexpr int STEPS = RG<T>::STEPS, LDW = ldw_of<T>();
  __shared__ LDS_ALIGN T Ws[D * LDW];
  __shared__ LnLds lns;
  lds_rows<T>(Ws, LDW, D, D, [&](int r) { return w + (int64_t)r * D; });
  stage_ln(lns, lnw, lnb);
  __syncthreads();
  const float* lw = lnw != nullptr ? lns.w : nullptr;
  const int64_t NN = N * N;
  const int ntiles = (int)((NN + 15) / 16), stride = gridDim.x * 4;
  const int l = threadIdx.x & 63, g = l >> 4;
  int t = grid_wave(4);
  if (t >= ntiles) return;
  const auto zrow_of = [&](int tt) -> int64_t {
    int64_t p = (int64_t)tt * 16 + (l & 15);
    if (p >= NN) return -1;
    if (trans) { const int64_t a = p / N; p = (p - a * N) * N + a; }
    return p;
  };
  const auto load = [&](int tt, typename RG<T>::frag (&xx)[1][STEPS], f4 (&zz)[1][8]) {
    RG<T>::load_row(xx[0], x_in + min((int64_t)tt * 16 + (l & 15), NN - 1) * D, g);
    const int64_t zr = zrow_of(tt);
    load_z_rows<1>(zz, [&](int) { return zr; }, z, accumulate);
  };
  typename RG<T>::frag x[1][STEPS];
  f4 zv[1][8];
  load(t, x, zv);
  for (; t < ntiles; t += stride) {
    typename RG<T>::frag xnext[1][STEPS];
    f4 znext[1][8];
    load(min(t + stride, ntiles - 1), xnext, znext);
    f4 y[1][8];
    zero_acc(y);
    mma_rows_grouped<T, 1, 8, 2>(y, x, Ws, LDW);
    const int64_t zr = zrow_of(t);
    resid_ln_apply<T, 1>(y, zv, [&](int) { return zr; }, z, lw, lns.b, eps, xn_next);
#pragma unroll
    for (int s = 0; s < STEPS; s++) x[0][s] = xnext[0][s];
#pragma unroll
    for (int cb = 0; cb < 8; cb++) zv[0][cb] = znext[0][cb];
  }
}

// ---------------------------------------------------------------- transition
// Hidden chunks of HCH units: h1^T, h2^T = fc1/fc2 chunk . xn^T (16-unit blocks), a = silu(h1) * h2 stays in the
// accumulator layout, which is already the B operand layout of out^T += fc3[:, chunk] . a^T (keys of the fp16 MFMA
// permuted as {4g .. 4g+3} u {16+4g .. 16+4g+3} within each 32-unit slice; fp32 steps take unit 4g + s).
template <typename T, int HCH>
__global__ __launch_bounds__(256) void transition_k(const T* __restrict__ xn, const T* __restrict__ w12,
                                                    const T* __restrict__ w3, float* __restrict__ z, int accumulate,
                                                    const float* __restrict__ lnw, const float* __restrict__ lnb,
                                                    float eps, T* __restrict__ xn_next, int64_t rows_total,
                                                    int hidden) {
  constexpr int RB = RowBlocks<T>::v, TM = 64 * RB, STEPS = RG<T>::STEPS, LDW = ldw_of<T>();
  constexpr int LDH = HCH + Pad<T>::v;
  constexpr int HB = HCH / 16;
  __shared__ LDS_ALIGN T W1s[HCH * LDW];
  __shared__ LDS_ALIGN T W2s[HCH * LDW];
  __shared__ LDS_ALIGN T W3s[D * LDH];
  const int64_t r0 = (int64_t)blockIdx.x * TM;
  const int wave = threadIdx.x >> 6, l = threadIdx.x & 63, g = l >> 4;
  typename RG<T>::frag x[RB][STEPS];
  int64_t row[RB];
#pragma unroll
  for (int rb = 0; rb < RB; rb++) {
    row[rb] = r0 + wave * 16 * RB + 16 * rb + (l & 15);
    RG<T>::load_row(x[rb], xn + (row[rb] < rows_total ? row[rb] : rows_total - 1) * D, g);
  }
  f4 out[RB][8];
  zero_acc(out);
  for (int h0 = 0; h0 < hidden; h0 += HCH) {
    __syncthreads();
    lds_rows<T>(W1s, LDW, HCH, D, [&](int r) { return w12 + (int64_t)(h0 + r) * D; });
    lds_rows<T>(W2s, LDW, HCH, D, [&](int r) { return w12 + (int64_t)(hidden + h0 + r) * D; });
    lds_rows<T>(W3s, LDH, D, HCH, [&](int r) { return w3 + (int64_t)r * hidden + h0; });
    __syncthreads();
    f4 a[RB][HB];
#pragma unroll
    for (int hb = 0; hb < HB; hb++) {
      f4 h1[RB][1], h2[RB][1];
      zero_acc(h1);
      zero_acc(h2);
      mma_rows<T, RB, 1>(h1, x, W1s + 16 * hb * LDW, LDW);
      mma_rows<T, RB, 1>(h2, x, W2s + 16 * hb * LDW, LDW);
#pragma unroll
      for (int rb = 0; rb < RB; rb++)
#pragma unroll
        for (int e = 0; e < 4; e++) a[rb][hb][e] = siluf_(h1[rb][0][e]) * h2[rb][0][e];
    }
    if constexpr (sizeof(T) == 2) {
#pragma unroll
      for (int m = 0; m < HB / 2; m++) {
        half8 bf[RB];
#pragma unroll
        for (int rb = 0; rb < RB; rb++)
#pragma unroll
          for (int e = 0; e < 4; e++) {
            bf[rb][e] = (half_t)a[rb][2 * m][e];
            bf[rb][4 + e] = (half_t)a[rb][2 * m + 1][e];
          }
#pragma unroll
        for (int ob = 0; ob < 8; ob++) {
          const T* wr = W3s + (16 * ob + (l & 15)) * LDH + 32 * m + 4 * g;
          const half4 lo = *reinterpret_cast<const half4*>(wr);
          const half4 hi = *reinterpret_cast<const half4*>(wr + 16);
          const half8 af = half8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
#pragma unroll
          for (int rb = 0; rb < RB; rb++)
            out[rb][ob] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af, bf[rb], out[rb][ob], 0, 0, 0);
        }
      }
    } else {
#pragma unroll
      for (int hb = 0; hb < HB; hb++)
#pragma unroll
        for (int s = 0; s < 4; s++)
#pragma unroll
          for (int ob = 0; ob < 8; ob++) {
            const float af = to_f(W3s[(16 * ob + (l & 15)) * LDH + 16 * hb + 4 * g + s]);
#pragma unroll
            for (int rb = 0; rb < RB; rb++)
              out[rb][ob] = __builtin_amdgcn_mfma_f32_16x16x4f32(af, a[rb][hb][s], out[rb][ob], 0, 0, 0);
          }
    }
  }
  resid_ln_rows<T, RB>(out, [&](int rb) -> int64_t { return row[rb] < rows_total ? row[rb] : -1; }, z, accumulate, lnw,
                       lnb, eps, xn_next);
}

// fp16 transition, persistent: TRW-wave workgroups (32 rows per wave, 2 waves per SIMD) walk tiles of 32 TRW rows.
// The hidden dimension streams through LDS in chunks of 32 units (fc1 and fc2 rows, fc3 columns: 24 KB; 4% faster
// than 64). Chunk q + 1 is loaded into registers while chunk q computes from LDS and is written to the other buffer
// afterwards, so a chunk costs one barrier and no exposed L2 latency; the buffer written in step q was last read in
// step q - 1, which every wave finished before the barrier of step q - 1. The chunk sequence runs on across tiles
// (the weights repeat), and the next tile's rows are loaded during the current tile's last chunk.
// TRW = 8: one workgroup per CU (large grids). TRW = 4: two per CU, whose barriers are independent, so one can run
// its row epilogue while the other computes; that wins at N = 400 (0.126 against 0.139 ms) and loses at N = 1000
// (0.687 against 0.656 ms), where the 256-row tile's fewer weight passes per row count more.
constexpr int TR_HCH = 32;

// AO: the ending-node attention's output stage runs in front (attn_out_rows): the kernel reads the attention core's
// output o (row of position (i, j) at (j, i) when trans) instead of xn and feeds LN(z + o W_o^T) with the
// transition's own norm to the chunk loop from registers; the epilogue recomputes z + o W_o^T from the tile's o and
// z rows (same bits) as its residual. Against the two kernels, the intermediate z and xn never go to memory.
struct AttnOutArgs {
  const half_t* o;
  const half_t* w_o;  // [128][128]
  int trans;
  int64_t n;  // tokens: rows_total = n * n
  const float* lnw;
  const float* lnb;
  float eps;
};

template <bool PB, int TRW, bool AO = false>
__global__ __launch_bounds__(64 * TRW, 8 / TRW) void transition_f16_k(const half_t* __restrict__ xn,
                                                                  const half_t* __restrict__ w12,
                                                                  const half_t* __restrict__ w3,
                                                                  float* __restrict__ z, int accumulate,
                                                                  const float* __restrict__ lnw,
                                                                  const float* __restrict__ lnb, float eps,
                                                                  half_t* __restrict__ xn_next, int64_t rows_total,
                                                                  int hidden, const half_t* __restrict__ pb_w,
                                                                  const float* __restrict__ pb_lnw,
                                                                  const float* __restrict__ pb_lnb, float pb_eps,
                                                                  half_t* __restrict__ pb_out, int pb_heads,
                                                                  AttnOutArgs ao, int64_t full_items,
                                                                  int part_rows) {
  using T = half_t;
  constexpr int RB = 2, STEPS = RG<T>::STEPS, LDW = ldw_of<T>(), LDH = TR_HCH + Pad<T>::v, HB = TR_HCH / 16;
  constexpr int TR_WAVES = TRW, TROWS = 16 * RB * TR_WAVES;
  constexpr int VPM = TR_HCH * 16 / (64 * TR_WAVES), VPT = 3 * VPM;  // 16-byte vectors of a chunk per thread
  constexpr int V3 = TR_HCH / 8;                                       // 16-byte vectors per fc3 row of a chunk
  static_assert(HB % 2 == 0 && VPM >= 1, "chunk shape");
  __shared__ LDS_ALIGN T W1s[2][TR_HCH * LDW];
  __shared__ LDS_ALIGN T W2s[2][TR_HCH * LDW];
  __shared__ LDS_ALIGN T W3s[2][D * LDH];
  // pair bias of the s track (PB): W' = W_pb with gamma_pb folded into its columns (heads past pb_heads zero), and
  // W_pb . beta_pb
  constexpr int LDP = D + 8;
  __shared__ LDS_ALIGN T Wpb[PB ? 16 * LDP : 8];
  __shared__ float Bpb[16];
  __shared__ LDS_ALIGN T Wo[AO ? D * LDW : 8];
  __shared__ LDS_ALIGN T Scr[AO ? TRW * 16 * SCR_P : 8];  // per wave: 16 rows of the attention stage's LayerNorm
  __shared__ LnLds lns[AO ? 2 : 1];                         // the next LayerNorm; [1]: the attention stage's
  const int t = threadIdx.x, l = t & 63, g = l >> 4;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const int nch = hidden / TR_HCH;
  // Work items: full_items tiles of TROWS rows, then the remaining rows in items of part_rows (a multiple of 32: whole
  // waves), so that the last round spreads over the grid instead of leaving most workgroups idle; in such an item
  // the waves past its rows stage chunks and meet the barriers but compute nothing.
  const int64_t part_base = full_items * TROWS;
  const int64_t ntiles =
      full_items + (rows_total > part_base ? (rows_total - part_base + part_rows - 1) / part_rows : 0);
  const auto item_base = [&](int64_t it) -> int64_t {
    return it < full_items ? it * TROWS : part_base + (it - full_items) * part_rows;
  };
  const auto item_rows = [&](int64_t it) -> int {
    return it < full_items ? TROWS : (int)min((int64_t)part_rows, rows_total - item_base(it));
  };
  int64_t tile = blockIdx.x;
  if (tile >= ntiles) return;  // whole workgroup
  if constexpr (AO) lds_rows<T>(Wo, LDW, D, D, [&](int r) { return ao.w_o + (int64_t)r * D; });
  stage_ln(lns[0], lnw, lnb);
  if constexpr (AO) stage_ln(lns[AO ? 1 : 0], ao.lnw, ao.lnb);
  const float* lw = lnw != nullptr ? lns[0].w : nullptr;
  const float* lb = lns[0].b;
  if constexpr (PB) {
    for (int e = t; e < 16 * D; e += 64 * TR_WAVES) {
      const int h = e >> 7, c = e & (D - 1);
      Wpb[h * LDP + c] = h < pb_heads ? (half_t)((float)pb_w[h * D + c] * pb_lnw[c]) : (half_t)0.0f;
    }
    if (t < 64) {  // 4 lanes per head, 32 channels each
      const int h = t >> 2, q = t & 3;
      float acc = 0.f;
      if (h < pb_heads)
        for (int c = 32 * q; c < 32 * q + 32; c++) acc += (float)pb_w[h * D + c] * pb_lnb[c];
      acc += __shfl_xor(acc, 1, 64);
      acc += __shfl_xor(acc, 2, 64);
      if (q == 0) Bpb[h] = acc;
    }
  }

  // chunk staging: vector v of thread t is element e = (v % VPM) * 64 TRW + t of matrix v / VPM (fc1, fc2: TR_HCH rows x
  // 16 vectors; fc3: 128 rows x V3 vectors of the chunk's TR_HCH columns)
  u32x4 pre[VPT];
  // element offsets of the thread's vectors in chunk 0 (chunk c adds c * TR_HCH * D in fc1/fc2, c * TR_HCH in fc3)
  uint32_t goff[VPT];
#pragma unroll
  for (int v = 0; v < VPT; v++) {
    const int m = v / VPM, e = (v % VPM) * (64 * TR_WAVES) + t;
    goff[v] = m < 2 ? (uint32_t)(m * hidden + (e >> 4)) * D + (e & 15) * 8 : (uint32_t)(e / V3) * hidden + (e % V3) * 8;
  }
  const auto gload = [&](int c) {
    const uint32_t h12 = (uint32_t)c * TR_HCH * D, h3 = (uint32_t)c * TR_HCH;
#pragma unroll
    for (int v = 0; v < VPT; v++)
      pre[v] = *reinterpret_cast<const u32x4*>(v < 2 * VPM ? w12 + (goff[v] + h12) : w3 + (goff[v] + h3));
  };
  // fc3 columns are stored permuted within each 32-column group: column 16 hi + 4 gg + e (gg < 4, e < 4) sits at
  // 8 gg + 4 hi + e, so the 8 columns lane group g multiplies (4 g .. 4 g + 3 and 16 + 4 g .. 16 + 4 g + 3, in
  // that k order) are one 16-byte read; a staged 16-byte vector (8 columns) splits into two 8-byte halves.
  const auto lstore = [&](int buf) {
#pragma unroll
    for (int v = 0; v < VPT; v++) {
      const int m = v / VPM, e = (v % VPM) * (64 * TR_WAVES) + t;
      if (m < 2) {
        T* dst = (m == 0 ? W1s[buf] : W2s[buf]) + (e >> 4) * LDW + (e & 15) * 8;
        *reinterpret_cast<u32x4*>(dst) = pre[v];
      } else {
        const int u = e % V3, ug = u & 3;  // vector u holds columns 8 u .. 8 u + 7
        T* dst = W3s[buf] + (e / V3) * LDH + 32 * (u >> 2) + 16 * (ug & 1) + 4 * (ug >> 1);
        *reinterpret_cast<uint2*>(dst) = uint2{pre[v][0], pre[v][1]};
        *reinterpret_cast<uint2*>(dst + 8) = uint2{pre[v][2], pre[v][3]};
      }
    }
  };
  const auto xload = [&](int64_t tl, typename RG<T>::frag (&xx)[RB][STEPS]) {
#pragma unroll
    for (int rb = 0; rb < RB; rb++) {
      const int64_t row = item_base(tl) + wave * 16 * RB + 16 * rb + (l & 15), rc = row < rows_total ? row : rows_total - 1;
      if constexpr (AO) {
        const int64_t orow = ao.trans ? (rc % ao.n) * ao.n + rc / ao.n : rc;
        RG<T>::load_row(xx[rb], ao.o + orow * D, g);
      } else {
        RG<T>::load_row(xx[rb], xn + rc * D, g);
      }
    }
  };

  typename RG<T>::frag x[RB][STEPS];
  xload(tile, x);
  gload(0);
  lstore(0);
  __syncthreads();
  gload(nch > 1 ? 1 : 0);
  int q = 0;  // chunks computed so far (LDS buffer parity)
  for (; tile < ntiles; tile += gridDim.x) {
    const int64_t base = item_base(tile);
    const int cnt = item_rows(tile), lrow0 = wave * 16 * RB + (l & 15);
    const bool wact = wave * 16 * RB < cnt;  // wave-uniform: the wave has rows in this item
    const int64_t row0 = base + lrow0;
    const auto zrow = [&](int rb) -> int64_t { return lrow0 + 16 * rb < cnt ? row0 + 16 * rb : -1; };
    if constexpr (AO) {
      if (wact)
        attn_out_rows<RB>(x, Wo, LDW, zrow, z, lns[AO ? 1 : 0].w, lns[AO ? 1 : 0].b, ao.eps, Scr + wave * 16 * SCR_P);
    }
    f4 out[RB][8];
    zero_acc(out);
    typename RG<T>::frag xnext[RB][STEPS];
    for (int c = 0; c < nch; c++, q++) {
      const int buf = q & 1;
      if (c == nch - 1) xload(min(tile + (int64_t)gridDim.x, ntiles - 1), xnext);
      if (wact) {
      f4 a[RB][HB];
#pragma unroll
      for (int hb = 0; hb < HB; hb++) {
        f4 h1[RB][1], h2[RB][1];
        zero_acc(h1);
        zero_acc(h2);
        mma_rows<T, RB, 1>(h1, x, W1s[buf] + 16 * hb * LDW, LDW);
        mma_rows<T, RB, 1>(h2, x, W2s[buf] + 16 * hb * LDW, LDW);
#pragma unroll
        for (int rb = 0; rb < RB; rb++)
#pragma unroll
          for (int e = 0; e < 4; e++) a[rb][hb][e] = siluf_(h1[rb][0][e]) * h2[rb][0][e];
      }
#pragma unroll
      for (int m = 0; m < HB / 2; m++) {
        half8 bf[RB];
#pragma unroll
        for (int rb = 0; rb < RB; rb++)
#pragma unroll
          for (int e = 0; e < 4; e++) {
            bf[rb][e] = (half_t)a[rb][2 * m][e];
            bf[rb][4 + e] = (half_t)a[rb][2 * m + 1][e];
          }
#pragma unroll
        for (int ob = 0; ob < 8; ob++) {
          const half8 af = *reinterpret_cast<const half8*>(W3s[buf] + (16 * ob + (l & 15)) * LDH + 32 * m + 8 * g);
#pragma unroll
          for (int rb = 0; rb < RB; rb++)
            out[rb][ob] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af, bf[rb], out[rb][ob], 0, 0, 0);
        }
      }
      }
      lstore(buf ^ 1);
      __syncthreads();
      gload(c + 2 < nch ? c + 2 : c + 2 - nch >= nch ? 0 : c + 2 - nch);
    }
    if (!wact) {
      // no rows here: the next item's rows (loaded during the last chunk) become current
    } else if constexpr (AO) {
      // the residual is z' = z + W_o o^T again, recomputed from the tile's o and z rows (x now holds the next
      // tile's o rows)
      const auto zvf = [&](int rb, f4(&zv)[8]) {
        typename RG<T>::frag x1[1][STEPS];
        {
          const int64_t rc = row0 + 16 * rb < rows_total ? row0 + 16 * rb : rows_total - 1;
          RG<T>::load_row(x1[0], ao.o + (ao.trans ? (rc % ao.n) * ao.n + rc / ao.n : rc) * D, g);
        }
        f4 zz[1][8];
        load_z_rows<1>(zz, [&](int) { return zrow(rb); }, z, 1);
        f4 y1[1][8];
        zero_acc(y1);
        mma_rows_grouped<T, 1, 8, 2>(y1, x1, Wo, LDW);
#pragma unroll
        for (int cb = 0; cb < 8; cb++) zv[cb] = y1[0][cb] + zz[0][cb];
      };
      if constexpr (PB) {
        resid_ln_pb_apply<RB>(out, zvf, zrow, z, lw, lb, eps, xn_next, Wpb, LDP, Bpb, pb_eps, pb_out, rows_total,
                              pb_heads);
      } else {
        f4 zv[RB][8];
#pragma unroll
        for (int rb = 0; rb < RB; rb++) zvf(rb, zv[rb]);
        resid_ln_apply<T, RB>(out, zv, zrow, z, lw, lb, eps, xn_next);
      }
    } else if constexpr (PB) {
      resid_ln_pb_rows<RB>(out, zrow, z, accumulate, lw, lb, eps, xn_next, Wpb, LDP, Bpb, pb_eps, pb_out,
                           rows_total, pb_heads);
    } else {
      resid_ln_rows<T, RB>(out, zrow, z, accumulate, lw, lb, eps, xn_next);
    }
#pragma unroll
    for (int rb = 0; rb < RB; rb++)
#pragma unroll
      for (int s2 = 0; s2 < STEPS; s2++) x[rb][s2] = xnext[rb][s2];
  }
}

}  // namespace

// ---------------------------------------------------------------- launchers

template <typename T, int HV>
static hipError_t tm_proj_hv(const void* xn, const void* w, const float* mask, float scale, int incoming, void* ab,
                             int64_t N, int64_t ld, int resident, hipStream_t st) {
  const int64_t ntiles = N * (ld / (HV * RunTile<T>::TW));  // ld is a multiple of 64
  if (ntiles >= (1LL << 30)) return hipErrorInvalidValue;  // tile indices are 32-bit in the kernel
  const dim3 grid((unsigned)std::min<int64_t>(resident, (ntiles + PROJ_WAVES - 1) / PROJ_WAVES));
  for (int c_lo = 0; c_lo < 2 * D; c_lo += proj_ch<T>()) {
    trimul_proj_k<T, HV><<<grid, 64 * PROJ_WAVES, 0, st>>>(static_cast<const T*>(xn), static_cast<const T*>(w), mask,
                                                          scale, incoming, static_cast<T*>(ab), N, ld, c_lo);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

template <typename T>
static hipError_t tm_proj(const void* xn, const void* w, const float* mask, float scale, int incoming, void* ab,
                          int64_t N, int64_t ld, hipStream_t st) {
  static int cache[kMaxDevices];
  // both tile forms have the same resources (the LDS weights and 8 waves set the occupancy)
  const int resident = resident_grid(trimul_proj_k<T, 2>, 64 * PROJ_WAVES, cache);
  if (resident <= 0) return hipErrorInvalidDevice;
  // rounds of full tiles on the resident waves, against rounds of half tiles (counted in full tiles, with 10% for
  // the half tile's own overhead)
  const int64_t waves = (int64_t)resident * PROJ_WAVES, full = N * (ld / (2 * RunTile<T>::TW));
  const int64_t r2 = (full + waves - 1) / waves, r1x2 = (2 * full + waves - 1) / waves;
  return 10 * r1x2 < 18 * r2 ? tm_proj_hv<T, 1>(xn, w, mask, scale, incoming, ab, N, ld, resident, st)
                             : tm_proj_hv<T, 2>(xn, w, mask, scale, incoming, ab, N, ld, resident, st);
}

hipError_t launch_trimul_proj(const void* xn, const void* w, const float* mask, float scale, int incoming, void* ab,
                              int dt, int64_t N, int64_t ld, hipStream_t st) {
  return dt == DT_F16 ? tm_proj<half_t>(xn, w, mask, scale, incoming, ab, N, ld, st)
                      : tm_proj<float>(xn, w, mask, scale, incoming, ab, N, ld, st);
}

template <typename T>
static hipError_t tm_tail(const void* o, const float* now, const float* nob, float eps_out, const void* w_po,
                          const void* xn, const void* w_go, float* z, int accumulate, const float* lnw,
                          const float* lnb, float eps_next, void* xn_next, int64_t N, int64_t ld, hipStream_t st) {
  constexpr int TM = 64 * RowBlocks<T>::v;
  const dim3 grid((unsigned)(N * ((ld + TM - 1) / TM)));
  trimul_tail_k<T><<<grid, 256, 0, st>>>(static_cast<const T*>(o), now, nob, eps_out, static_cast<const T*>(w_po),
                                         static_cast<const T*>(xn), static_cast<const T*>(w_go), z, accumulate, lnw,
                                         lnb, eps_next, static_cast<T*>(xn_next), N, ld);
  return hipGetLastError();
}

static hipError_t tm_tail_f16(const void* o, const float* now, const float* nob, float eps_out, const void* w_po,
                              const void* xn, const void* w_go, float* z, int accumulate, const float* lnw,
                              const float* lnb, float eps_next, void* xn_next, int64_t N, int64_t ld, hipStream_t st) {
  static int cache[kMaxDevices];
  const int resident = resident_grid(trimul_tail_f16_k, 64 * TAIL_WAVES, cache);
  if (resident <= 0) return hipErrorInvalidDevice;
  const int64_t ntiles = N * tail_tiles_per_row(N);  // the last tile of a row ends at ld (ld = N rounded up to 64)
  if (ntiles >= (1LL << 30)) return hipErrorInvalidValue;  // tile indices are 32-bit in the kernel
  const dim3 grid((unsigned)std::min<int64_t>(resident, (ntiles + TAIL_WAVES - 1) / TAIL_WAVES));
  trimul_tail_f16_k<<<grid, 64 * TAIL_WAVES, 0, st>>>(static_cast<const half_t*>(o), now, nob, eps_out,
                                                      static_cast<const half_t*>(w_po), static_cast<const half_t*>(xn),
                                                      static_cast<const half_t*>(w_go), z, accumulate, lnw, lnb,
                                                      eps_next, static_cast<half_t*>(xn_next), N, ld);
  return hipGetLastError();
}

hipError_t launch_trimul_tail(const void* o, const float* now, const float* nob, float eps_out, const void* w_po,
                              const void* xn, const void* w_go, float* z, int accumulate, const float* lnw,
                              const float* lnb, float eps_next, void* xn_next, int dt, int64_t N, int64_t ld,
                              hipStream_t st) {
  if (dt == DT_F16 && (int64_t)D * N * ld < (1LL << 31))
    return tm_tail_f16(o, now, nob, eps_out, w_po, xn, w_go, z, accumulate, lnw, lnb, eps_next, xn_next, N, ld, st);
  return dt == DT_F16 ? tm_tail<half_t>(o, now, nob, eps_out, w_po, xn, w_go, z, accumulate, lnw, lnb, eps_next,
                                        xn_next, N, ld, st)
                      : tm_tail<float>(o, now, nob, eps_out, w_po, xn, w_go, z, accumulate, lnw, lnb, eps_next,
                                       xn_next, N, ld, st);
}

template <typename T>
static hipError_t ta_proj(const void* xn, const void* w, int trans, float q_scale, float b_scale, void* qkg, void* vt,
                          void* tb, int64_t N, int64_t ldk, int H, int C, hipStream_t st) {
  if (H * C != D || H > 16 || C % 8) return hipErrorInvalidValue;
  static int cache[kMaxDevices];
  const int resident = resident_grid(triattn_proj_k<T>, 64 * ATTN_PROJ_WAVES, cache);
  if (resident <= 0) return hipErrorInvalidDevice;
  const int64_t ntiles = N * (ldk / RunTile<T>::TW);  // ldk is a multiple of 64
  if (ntiles >= (1LL << 30)) return hipErrorInvalidValue;  // tile indices are 32-bit in the kernel
  const dim3 grid((unsigned)std::min<int64_t>(resident, (ntiles + ATTN_PROJ_WAVES - 1) / ATTN_PROJ_WAVES));
  const int bounds[3] = {0, sizeof(T) == 2 ? 4 * D + 16 : 2 * D, 4 * D + 16};
  for (int p = 0; p < (sizeof(T) == 2 ? 1 : 2); p++) {
    triattn_proj_k<T><<<grid, 64 * ATTN_PROJ_WAVES, 0, st>>>(
        static_cast<const T*>(xn), static_cast<const T*>(w), trans, q_scale, b_scale, static_cast<T*>(qkg),
        static_cast<T*>(vt), static_cast<T*>(tb), N, ldk, H, C, bounds[p], bounds[p + 1]);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

hipError_t launch_triattn_proj(const void* xn, const void* w, int trans, float q_scale, float b_scale, void* qkg,
                               void* vt, void* tb, int dt, int64_t N, int64_t ldk, int H, int C, hipStream_t st) {
  return dt == DT_F16 ? ta_proj<half_t>(xn, w, trans, q_scale, b_scale, qkg, vt, tb, N, ldk, H, C, st)
                      : ta_proj<float>(xn, w, trans, q_scale, b_scale, qkg, vt, tb, N, ldk, H, C, st);
}

template <typename T>
static hipError_t lrl(const void* x, const void* w, int trans, float* z, int accumulate, const float* lnw,
                      const float* lnb, float eps, void* xn_next, int64_t N, hipStream_t st) {
  static int cache[kMaxDevices];
  const int resident = resident_grid(linear_resid_ln_k<T>, 256, cache);
  if (resident <= 0) return hipErrorInvalidDevice;
  const int64_t waves = (N * N + 15) / 16;
  if (waves >= (1LL << 30)) return hipErrorInvalidValue;  // tile indices are 32-bit in the kernel
  const dim3 grid((unsigned)std::min<int64_t>(resident, (waves + 3) / 4));
  linear_resid_ln_k<T><<<grid, 256, 0, st>>>(static_cast<const T*>(x), static_cast<const T*>(w), trans, z, accumulate,
                                             lnw, lnb, eps, static_cast<T*>(xn_next), N);
  return hipGetLastError();
}

hipError_t launch_linear_resid_ln(const void* x, const void* w, int trans, float* z, int accumulate,
                                  const float* lnw, const float* lnb, float eps, void* xn_next, int dt, int64_t N,
                                  hipStream_t st) {
  return dt == DT_F16 ? lrl<half_t>(x, w, trans, z, accumulate, lnw, lnb, eps, xn_next, N, st)
                      : lrl<float>(x, w, trans, z, accumulate, lnw, lnb, eps, xn_next, N, st);
}

template <typename T, int HCH>
static hipError_t trans_t(const void* xn, const void* w12, const void* w3, float* z, int accumulate, const float* lnw,
                          const float* lnb, float eps, void* xn_next, int64_t rows, int hidden, hipStream_t st) {
  if (hidden % HCH) return hipErrorInvalidValue;
  constexpr int TM = 64 * RowBlocks<T>::v;
  const dim3 grid((unsigned)((rows + TM - 1) / TM));
  transition_k<T, HCH><<<grid, 256, 0, st>>>(static_cast<const T*>(xn), static_cast<const T*>(w12),
                                             static_cast<const T*>(w3), z, accumulate, lnw, lnb, eps,
                                             static_cast<T*>(xn_next), rows, hidden);
  return hipGetLastError();
}

template <bool PB, int TRW, bool AO = false>
static hipError_t trans_f16_w(const void* xn, const void* w12, const void* w3, float* z, int accumulate,
                              const float* lnw, const float* lnb, float eps, void* xn_next, int64_t rows, int hidden,
                              const void* pb_w, const float* pb_lnw, const float* pb_lnb, float pb_eps, void* pb_out,
                              int pb_heads, hipStream_t st, const AttnOutArgs& ao = AttnOutArgs{}) {
  static int cache[kMaxDevices];
  const int resident = resident_grid(transition_f16_k<PB, TRW, AO>, 64 * TRW, cache);
  if (resident <= 0) return hipErrorInvalidDevice;
  if (rows <= 0) return hipSuccess;
  // whole rounds of 32 TRW-row tiles over the resident grid, then the remaining rows split evenly over it in items
  // of whole waves (32 rows each)
  const int64_t trows = 32 * TRW, full_items = rows / (trows * resident) * resident, rem = rows - full_items * trows;
  const int64_t part = rem > 0 ? ((rem + resident - 1) / resident + 31) / 32 * 32 : trows;
  const int64_t nitems = full_items + (rem + part - 1) / part;
  const dim3 grid((unsigned)std::min<int64_t>(resident, nitems));
  transition_f16_k<PB, TRW, AO><<<grid, 64 * TRW, 0, st>>>(
      static_cast<const half_t*>(xn), static_cast<const half_t*>(w12), static_cast<const half_t*>(w3), z, accumulate,
      lnw, lnb, eps, static_cast<half_t*>(xn_next), rows, hidden, static_cast<const half_t*>(pb_w), pb_lnw, pb_lnb,
      pb_eps, static_cast<half_t*>(pb_out), pb_heads, ao, full_items, (int)part);
  return hipGetLastError();
}

// rows below 400,000 (N = 632 for a pair stack) take the two-workgroup form
template <bool PB>
static hipError_t trans_f16(const void* xn, const void* w12, const void* w3, float* z, int accumulate,
                            const float* lnw, const float* lnb, float eps, void* xn_next, int64_t rows, int hidden,
                            const void* pb_w, const float* pb_lnw, const float* pb_lnb, float pb_eps, void* pb_out,
                            int pb_heads, hipStream_t st) {
  return rows < 400000 ? trans_f16_w<PB, 4>(xn, w12, w3, z, accumulate, lnw, lnb, eps, xn_next, rows, hidden, pb_w,
                                            pb_lnw, pb_lnb, pb_eps, pb_out, pb_heads, st)
                       : trans_f16_w<PB, 8>(xn, w12, w3, z, accumulate, lnw, lnb, eps, xn_next, rows, hidden, pb_w,
                                            pb_lnw, pb_lnb, pb_eps, pb_out, pb_heads, st);
}

hipError_t launch_transition(const void* xn, const void* w12, const void* w3, float* z, int accumulate,
                             const float* lnw, const float* lnb, float eps, void* xn_next, int dt, int64_t rows,
                             int hidden, hipStream_t st) {
  if (dt == DT_F16 && hidden % TR_HCH == 0 && (int64_t)2 * hidden * D < (1LL << 31))
    return trans_f16<false>(xn, w12, w3, z, accumulate, lnw, lnb, eps, xn_next, rows, hidden, nullptr, nullptr,
                            nullptr, 0.f, nullptr, 0, st);
  return dt == DT_F16 ? trans_t<half_t, 64>(xn, w12, w3, z, accumulate, lnw, lnb, eps, xn_next, rows, hidden, st)
                      : trans_t<float, 32>(xn, w12, w3, z, accumulate, lnw, lnb, eps, xn_next, rows, hidden, st);
}

// Transition + the s track's pair bias from the updated z: the fp16 kernel computes it in its epilogue; otherwise
// the pair-bias kernel runs after the transition (same result definition).
hipError_t launch_transition_pb(const void* xn, const void* w12, const void* w3, float* z, int accumulate,
                                const float* lnw, const float* lnb, float eps, void* xn_next, const void* pb_w,
                                const float* pb_lnw, const float* pb_lnb, float pb_eps, void* pb_out, int pb_heads,
                                int dt, int64_t rows, int hidden, hipStream_t st) {
  if (pb_heads < 1 || pb_heads > 16) return hipErrorInvalidValue;
  if (dt == DT_F16 && hidden % TR_HCH == 0 && (int64_t)2 * hidden * D < (1LL << 31))
    return trans_f16<true>(xn, w12, w3, z, accumulate, lnw, lnb, eps, xn_next, rows, hidden, pb_w, pb_lnw, pb_lnb,
                           pb_eps, pb_out, pb_heads, st);
  const hipError_t e = launch_transition(xn, w12, w3, z, accumulate, lnw, lnb, eps, xn_next, dt, rows, hidden, st);
  if (e != hipSuccess) return e;
  return launch_pair_bias(z, pb_lnw, pb_lnb, pb_eps, pb_w, pb_out, dt, rows, pb_heads, st);
}

// The ending-node attention's output stage fused in front of the transition (fp16): one 8-wave workgroup per CU
// (its LDS holds W_o and the LayerNorm scratch next to the weight chunks).
hipError_t launch_attn_out_transition(const void* o, const void* w_o, int trans, const float* ln_w, const float* ln_b,
                                      float ln_eps, const void* w12, const void* w3, float* z, const float* next_w,
                                      const float* next_b, float next_eps, void* xn_next, const void* pb_w,
                                      const float* pb_lnw, const float* pb_lnb, float pb_eps, void* pb_out,
                                      int pb_heads, int64_t N, int hidden, hipStream_t st) {
  if (hidden % TR_HCH || hidden < 2 * TR_HCH || (int64_t)2 * hidden * D >= (1LL << 31) || N < 1)
    return hipErrorInvalidValue;
  const AttnOutArgs ao{static_cast<const half_t*>(o), static_cast<const half_t*>(w_o), trans, N, ln_w, ln_b, ln_eps};
  const int64_t rows = N * N;
  if (pb_w != nullptr) {
    if (pb_heads < 1 || pb_heads > 16) return hipErrorInvalidValue;
    return trans_f16_w<true, 8, true>(nullptr, w12, w3, z, 1, next_w, next_b, next_eps, xn_next, rows, hidden, pb_w,
                                      pb_lnw, pb_lnb, pb_eps, pb_out, pb_heads, st, ao);
  }
  return trans_f16_w<false, 8, true>(nullptr, w12, w3, z, 1, next_w, next_b, next_eps, xn_next, rows, hidden, nullptr,
                                     nullptr, nullptr, 0.f, nullptr, 0, st, ao);
}

}  // namespace bzpf
