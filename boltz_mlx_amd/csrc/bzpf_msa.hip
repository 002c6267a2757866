// MSA-block pair kernels (fp32 operands and fp32-accurate reductions, the reference's numerics policy for the
// reductions over MSA rows and tokens):
//   opm_split   : the masked operands mask[s][n] ab[s][n][ch] as bf16 part planes for opm_outer;
//   opm_outer   : z[(i - i_base) N + j][c 32 + d] = sum_s mask[s][i] mask[s][j] a[s][i][c] b[s][j][d] / max(num, 1)
//                 with num[i][j] = sum_s mask[s][i] mask[s][j] given (mask^T mask, one small GEMM) and
//                 a | b = ab[s][i][0:32] | ab[s][j][32:64]
//                 (OuterProductMean's outer sum, boltz_mlx/layers/outer_product_mean.py:37-45,
//                 boltz_mlx/kernels_msa.py:292-343), stored fp16 (the proj_o GEMM's operand) or fp32;
//   pwa_softmax : w[h][i][j] = softmax_j(logit[h][i][j] + (1 - pair_mask[i][j]) * -inf), rows padded with zeros
//                 to ldw (boltz_mlx/layers/pair_averaging.py:43-49, kernels_msa.py:461-500);
//   pwa_wsplit  : the weights w as bf16 part chunks for pwa_avg;
//   pwa_avg     : out[s][i][h 32 + d] = sigmoid(g[s][i][h 32 + d]) * sum_j w[h][i][j] v[s][j][h 32 + d]
//                 (pair_averaging.py:50-57, kernels_msa.py:620-653).
#include "bzpf_common.h"
#include "bzpf_kernels.h"
#include "bzpf_x3.h"

namespace bzpf {

namespace {

// Both reductions run on the bf16 matrix cores at fp32 accuracy (three exact bf16 parts per fp32 operand, six part
// products: bzpf_x3.h). A 256-thread workgroup computes a 128 x 128 tile over K stages of 16 (one MFMA K-step), two
// workgroups per CU. The outer sum takes both operands split beforehand (one pass over the MSA) and copies them
// straight into LDS; the weighted average takes its weights split beforehand (pwa_wsplit_k) as register fragments
// and splits the v columns in its loop.

// ---------------------------------------------------------------- outer product mean
// The outer sum takes its operands already split: a pass over the MSA writes the masked values
// x = mask[s][n] ab[s][n][ch] (the fp32 products) as their three bf16 parts, in 1 KB chunks that the outer sum
// copies straight into LDS (buffer_load ... lds), so its loop holds no staging registers and no split work.
// Chunk (g, n, p, h) at byte ((g N + n) 6 + 2 p + h) 1024 holds part p of channels 32 h .. 32 h + 31 of token n
// (h = 0: a, h = 1: b) over MSA rows 16 g .. 16 g + 15: 32 rows (channel c) of 16 bf16 (k = s - 16 g), zeros for
// s >= S.
constexpr int OPM_CHUNK = 1024, OPM_TOKB = 6 * OPM_CHUNK;

// A workgroup takes stage g of tokens 2 x .. 2 x + 1: thread (token t / 128, channel ch = (t / 2) % 64,
// kh = t % 2) takes MSA rows 16 g + 8 kh .. + 7 of channel ch and stores each part's 8 values as 16 bytes, so a
// wave's store of one part fills a 1 KB chunk.
__global__ __launch_bounds__(256) void opm_split_k(const float* __restrict__ ab, int64_t ld_ab,
                                                   const float* __restrict__ mask, __bf16* __restrict__ planes, int S,
                                                   int N) {
  const int t = threadIdx.x, n = 2 * (int)blockIdx.x + (t >> 7), g = (int)blockIdx.y;
  const int ch = (t >> 1) & 63, kh = t & 1;
  if (n >= N) return;  // the second half of the last workgroup for odd N (no barriers here)
  float x[8];
#pragma unroll
  for (int e = 0; e < 8; e++) {
    const int s = 16 * g + 8 * kh + e;
    const int sc = min(s, S - 1);
    const float v = ab[((int64_t)sc * N + n) * ld_ab + ch], m = mask[(int64_t)sc * N + n];
    x[e] = s < S ? v * m : 0.0f;
  }
  Pair3 q[4];
#pragma unroll
  for (int e = 0; e < 4; e++) q[e] = split3_pair(x[2 * e], x[2 * e + 1]);
  char* base = reinterpret_cast<char*>(planes) + ((int64_t)g * N + n) * OPM_TOKB + (ch >> 5) * OPM_CHUNK +
               (ch & 31) * 32 + 16 * kh;
#pragma unroll
  for (int p = 0; p < 3; p++)
    *reinterpret_cast<uint4*>(base + 2 * p * OPM_CHUNK) = uint4{q[0].p[p], q[1].p[p], q[2].p[p], q[3].p[p]};
}

// Workgroup tile: tokens i0 .. i0 + 3 (A rows (i, c) = 32 (i - i0) + c) x j0 .. j0 + 3 (B columns (j, d)), K = MSA
// rows s in stages of 16; a stage is 24 chunks (A: parts 0..2 of the a halves of tokens i0 .., B: of the b halves of
// tokens j0 ..), 24 KB of LDS, three stages in flight (two workgroups per CU). In LDS, row c of a chunk keeps its two
// 16-byte halves swapped when (c / 4) is odd, so the fragment reads (8 lanes on 8 consecutive rows per pass) hit
// distinct banks; each lane of a load picks the global half that lands there.
template <typename TO>
__global__ __launch_bounds__(256, 2) void opm_outer_k(const __bf16* __restrict__ planes, const float* __restrict__ num,
                                                      TO* __restrict__ out, int G, int N, int i_base, int n_i) {
  constexpr int NS = 3, STAGE = 24 * OPM_CHUNK, LPW = 6;  // load instructions per wave per stage
  __shared__ __attribute__((aligned(1024))) char lds[NS * STAGE];
  const int t = threadIdx.x, l = t & 63, r32 = l & 31, hl = l >> 5;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const int wm = wave >> 1, wn = wave & 1;
  const int i0 = i_base + 4 * (int)blockIdx.y, j0 = 4 * (int)blockIdx.x;
  const int i_end = min(i_base + n_i, N);
  // load v of this wave fills chunk q = wave + 4 v of the stage: q < 12 is A part q / 4 of token i0 + q % 4, else
  // B part (q - 12) / 4 of token j0 + q % 4 (tokens past the range load the last one; their outputs are not stored)
  int voff[LPW];
#pragma unroll
  for (int v = 0; v < LPW; v++) {
    const int q = wave + 4 * v, isb = q >= 12, p = (q % 12) / 4, tt = q % 4;
    const int n = isb ? min(j0 + tt, N - 1) : min(i0 + tt, i_end - 1);
    voff[v] = (n * 6 + 2 * p + isb) * OPM_CHUNK + (l >> 1) * 32 + 16 * ((l & 1) ^ ((l >> 3) & 1));
  }
  constexpr int RSRC_CFG = 0x00020000;
  auto issue = [&](int st, int slot) {
    st = min(st, G - 1);  // issues past the last stage reload it into a slot that is never read
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(reinterpret_cast<const char*>(planes) + (int64_t)st * N * OPM_TOKB), 0, N * OPM_TOKB, RSRC_CFG);
#pragma unroll
    for (int v = 0; v < LPW; v++)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          rs, (__attribute__((address_space(3))) void*)(lds + slot * STAGE + (wave + 4 * v) * OPM_CHUNK), 16,
          voff[v], 0, 0, 0);
  };
  // fragments: part p of A rows 64 wm + 32 bm + r32 (chunk p * 4 + 2 wm + bm, row r32) and of B columns
  // 64 wn + 32 bn + r32 (chunk 12 + p * 4 + 2 wn + bn), k = 8 hl .. 8 hl + 7
  const int fro = r32 * 32 + 16 * (hl ^ ((r32 >> 2) & 1));
  typedef bf16x8 Frag[2][3];
  Frag fa0, fb0, fa1, fb1;  // two sets, named (an array indexed by the stage parity would live in scratch)
  auto read = [&](Frag& fa, Frag& fb, int slot) {
    const char* base = lds + slot * STAGE + fro;
#pragma unroll
    for (int x = 0; x < 2; x++)
#pragma unroll
      for (int p = 0; p < 3; p++) {
        fa[x][p] = *reinterpret_cast<const bf16x8*>(base + (p * 4 + 2 * wm + x) * OPM_CHUNK);
        fb[x][p] = *reinterpret_cast<const bf16x8*>(base + (12 + p * 4 + 2 * wn + x) * OPM_CHUNK);
      }
  };
  f16x acc[2][2];
#pragma unroll
  for (int a = 0; a < 2; a++)
#pragma unroll
    for (int b = 0; b < 2; b++)
#pragma unroll
      for (int e = 0; e < 16; e++) acc[a][b][e] = 0.0f;
  constexpr int YOUNGER = (NS - 2) * LPW;  // loads of later stages in flight when a stage is waited for
  constexpr int WAIT = (YOUNGER & 15) | ((YOUNGER >> 4) << 14) | (0x7 << 4) | (0xF << 8);  // vmcnt only
#pragma unroll
  for (int p = 0; p < NS - 1; p++) issue(p, p);
  __builtin_amdgcn_s_waitcnt(WAIT);
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_sched_barrier(0);
  issue(NS - 1, NS - 1);
  read(fa0, fb0, 0);
  auto step = [&](int st, const Frag& ca, const Frag& cb, Frag& na, Frag& nb) {
    if (st + 1 < G) {
      // this wave's reads of slot st % NS are done and stage st + 1 has landed; after the barrier the slot takes
      // stage st + NS, and the fragments of stage st + 1 are read while stage st computes
      __builtin_amdgcn_s_waitcnt(WAIT & ~(0xF << 8));  // vmcnt as above, lgkmcnt(0)
      __builtin_amdgcn_s_barrier();
      __builtin_amdgcn_sched_barrier(0);
      issue(st + NS, st % NS);
      read(na, nb, (st + 1) % NS);
    }
#pragma unroll
    for (int bm = 0; bm < 2; bm++)
#pragma unroll
      for (int bn = 0; bn < 2; bn++) acc[bm][bn] = mfma_parts6(ca[bm], cb[bn], acc[bm][bn]);
  };
  for (int st = 0; st < G; st += 2) {
    step(st, fa0, fb0, fa1, fb1);
    if (st + 1 < G) step(st + 1, fa1, fb1, fa0, fb0);
  }
  // block (bm, bn): tokens i0 + 2 wm + bm and j0 + 2 wn + bn (wave-uniform); register r holds channel
  // c = 8 (r / 4) + 4 hl + r % 4 of a, lane r32 channel d = r32 of b
  float cnt[2][2];
#pragma unroll
  for (int bm = 0; bm < 2; bm++)
#pragma unroll
    for (int bn = 0; bn < 2; bn++) {
      const int i = min(i0 + 2 * wm + bm, N - 1), j = min(j0 + 2 * wn + bn, N - 1);
      cnt[bm][bn] = fmaxf(num[(int64_t)i * N + j], 1.0f);
    }
#pragma unroll
  for (int bm = 0; bm < 2; bm++)
#pragma unroll
    for (int bn = 0; bn < 2; bn++) {
      const int i = i0 + 2 * wm + bm, j = j0 + 2 * wn + bn;
      if (i >= i_end || j >= N) continue;  // wave-uniform
      TO* op = out + ((int64_t)(i - i_base) * N + j) * 1024 + r32;
#pragma unroll
      for (int r = 0; r < 16; r++) {
        const int c = 8 * (r >> 2) + 4 * hl + (r & 3);
        op[c * 32] = (TO)(acc[bm][bn][r] / cnt[bm][bn]);
      }
    }
}

// ---------------------------------------------------------------- pair-weighted averaging
// One wave per row (h, i): x_j = logit + (1 - pm[i][j]) * -inf in fp32, softmax over j < N, zeros for N <= j < ldw.
__global__ __launch_bounds__(256) void pwa_softmax_k(const float* __restrict__ logits, const float* __restrict__ pm,
                                                     float inf, float* __restrict__ w, int N, int64_t ldw,
                                                     int64_t rows) {
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int l = threadIdx.x & 63;
  const int64_t i = row % N;
  const float* x = logits + row * N;
  const float* mr = pm + i * N;
  float mx = -INFINITY;
  for (int j = l; j < N; j += 64) mx = fmaxf(mx, x[j] + (1.0f - mr[j]) * -inf);
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
  float sum = 0.0f;
  for (int j = l; j < N; j += 64) sum += expf(x[j] + (1.0f - mr[j]) * -inf - mx);
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) sum += __shfl_xor(sum, o);
  const float inv = 1.0f / sum;
  float* wr = w + row * ldw;
  for (int j = l; j < ldw; j += 64) wr[j] = j < N ? expf(x[j] + (1.0f - mr[j]) * -inf - mx) * inv : 0.0f;
}

// The weights' parts for the average: chunk (h, ib, jg, p) at byte (((h NIB + ib) NJG + jg) 3 + p) 1024
// (NIB = ceil(N / 32), NJG = ldw / 16 rounded up to even) holds part p of w[h][i][j] for rows i = 32 ib .. + 31 and
// tokens j = 16 jg .. + 15 (zeros past N and past ldw), as 32 rows of 16 bf16, so a wave's 16-byte loads of one
// chunk are one contiguous KB. A workgroup takes one (h, ib, jg) chunk triple: thread (row t / 8, token pair t % 8).
__global__ __launch_bounds__(256) void pwa_wsplit_k(const float* __restrict__ w, int64_t ldw, __bf16* __restrict__ wp,
                                                    int N, int nib, int njg) {
  const int jg = (int)blockIdx.x, ib = (int)blockIdx.y, h = (int)blockIdx.z, t = threadIdx.x;
  const int row = t >> 3, jp = t & 7, i = 32 * ib + row;
  float2 x = {0.0f, 0.0f};
  if (i < N && 16 * jg < ldw) x = *reinterpret_cast<const float2*>(w + ((int64_t)h * N + i) * ldw + 16 * jg + 2 * jp);
  const Pair3 q = split3_pair(x.x, x.y);
  char* base = reinterpret_cast<char*>(wp) + (((int64_t)h * nib + ib) * njg + jg) * 3 * 1024 + row * 32 + 4 * jp;
#pragma unroll
  for (int p = 0; p < 3; p++) *reinterpret_cast<uint32_t*>(base + p * 1024) = q.p[p];
}

// The average, on the three-part bf16 scheme above. Workgroup tile: rows i0 .. i0 + 127 of head h (A = w[h], k = j)
// x four MSA rows s0 .. s0 + 3 times the head's 32 channels (B columns (s, d)); a stage is 16 tokens j. Wave w takes
// rows 32 w .. + 31 against all 128 columns (1 x 4 blocks, block bn = MSA row s0 + bn). The A parts come split from
// pwa_wsplit_k (a weight serves every MSA-row tile, so it is split once, not once per tile) and a wave's A fragments
// are loaded from them straight into registers, two stages ahead (each wave reads rows no other wave reads). The v
// rows arrive d-contiguous, so a thread takes two consecutive tokens of 4 channels (two stages ahead in registers),
// splits them and stores each channel's pair of parts as one dword of the K-contiguous B planes (LDS
// double-buffered, one barrier per stage, two workgroups per CU).
__global__ __launch_bounds__(256, 2) void pwa_avg_k(const __bf16* __restrict__ wp, int nib, int njg,
                                                    const float* __restrict__ v, int64_t ldv,
                                                    const float* __restrict__ g, int64_t ldg, float* __restrict__ out,
                                                    int64_t ldo, int S, int N) {
  __shared__ LDS_ALIGN __bf16 Bs[2][3 * PLANE];
  const int t = threadIdx.x, wave = t >> 6, l = t & 63, r32 = l & 31, hl = l >> 5;
  const int i0 = 128 * (int)blockIdx.x, s0 = 4 * (int)blockIdx.y, h = (int)blockIdx.z;
  const int nst = njg;  // even (the split weights are zero in a padding stage)
  // A fragment p of stage st: chunk (h, ib = 4 blockIdx.x + wave (clamped to the last; rows past N are zero), st, p),
  // lane bytes 32 r32 + 16 hl
  const int ib = min(4 * (int)blockIdx.x + wave, nib - 1);
  const char* wa = reinterpret_cast<const char*>(wp) + ((int64_t)h * nib + ib) * njg * 3072 + r32 * 32 + 16 * hl;
  typedef bf16x8 AFrag[3];
  AFrag fa0, fa1;  // two named sets (an array indexed by the stage parity would live in scratch)
  auto aload = [&](AFrag& fa, int st) {
    st = min(st, nst - 1);  // loads past the last stage repeat it (never used)
#pragma unroll
    for (int p = 0; p < 3; p++) fa[p] = *reinterpret_cast<const bf16x8*>(wa + ((int64_t)st * 3 + p) * 1024);
  };
  // B item of thread t: MSA row s0 + t / 64, tokens 2 (t % 8) and 2 (t % 8) + 1, channels 4 ((t / 8) % 8) .. + 3.
  // Loads without conditions: MSA rows past S read the last valid one (their outputs are not stored), and tokens
  // past N (and past the last stage) read token N - 1's v, which meets zero weights there.
  const int bp = t & 7, bq = (t >> 3) & 7, bs = t >> 6;
  const int sb = min(s0 + bs, S - 1);
  f4 rb0[2], rb1[2];
  auto gload = [&](f4 (&rb)[2], int stage) {
#pragma unroll
    for (int b = 0; b < 2; b++) {
      const int key = min(stage * KS + 2 * bp + b, N - 1);
      rb[b] = *reinterpret_cast<const f4*>(v + ((int64_t)sb * N + key) * ldv + 32 * h + 4 * bq);
    }
  };
  auto lstore = [&](const f4 (&rb)[2], int buf) {
#pragma unroll
    for (int q = 0; q < 4; q++) {
      const Pair3 x = split3_pair(rb[0][q], rb[1][q]);
      __bf16* dst = Bs[buf] + (32 * bs + 4 * bq + q) * LDP + 2 * bp;
#pragma unroll
      for (int p = 0; p < 3; p++) *reinterpret_cast<uint32_t*>(dst + p * PLANE) = x.p[p];
    }
  };
  f16x acc[4];
#pragma unroll
  for (int b = 0; b < 4; b++)
#pragma unroll
    for (int e = 0; e < 16; e++) acc[b][e] = 0.0f;
  // one stage: B fragments of columns 32 bn + r32 from the B planes, the six part products per block
  auto compute = [&](const AFrag& fa, const __bf16* Bb) {
    bf16x8 fb[4][3];
#pragma unroll
    for (int bn = 0; bn < 4; bn++)
#pragma unroll
      for (int p = 0; p < 3; p++)
        fb[bn][p] = *reinterpret_cast<const bf16x8*>(Bb + p * PLANE + (32 * bn + r32) * LDP + 8 * hl);
#pragma unroll
    for (int bn = 0; bn < 4; bn++) acc[bn] = mfma_parts6(fa, fb[bn], acc[bn]);
  };
  // the prologue issues its loads in the steps' order (B of stage 1, A of 1, B of 2, then A of 2 in step 0), so the
  // first steps wait for the same loads as the later ones
  aload(fa0, 0);
  gload(rb0, 0);
  lstore(rb0, 0);
  __syncthreads();
  __builtin_amdgcn_sched_barrier(0);
  gload(rb0, 1);
  aload(fa1, 1);
  gload(rb1, 2);
  __builtin_amdgcn_sched_barrier(0);
  // step st: computes stage st (A set st & 1, B buffer st & 1) and then loads A of stage st + 2 into the set; stores
  // B of stage st + 1 (in rn) into the other buffer, whose last reader (stage st - 1) every wave finished before the
  // previous barrier (past the last stage: a buffer nobody reads); after the barrier rn takes B of stage st + 3
  // (the scheduling barriers keep each step's work on its side of the barrier: a split hoisted from the next step
  // would wait for that step's B loads, the youngest)
  auto step = [&](int st, AFrag& fa, f4 (&rn)[2]) {
    compute(fa, Bs[st & 1]);
    aload(fa, st + 2);
    lstore(rn, (st + 1) & 1);
    __syncthreads();
    __builtin_amdgcn_sched_barrier(0);
    gload(rn, st + 3);
    __builtin_amdgcn_sched_barrier(0);
  };
  for (int st = 0; st < nst; st += 2) {
    step(st, fa0, rb0);
    step(st + 1, fa1, rb1);
  }
  // block bn register r: row i0 + 32 wave + 8 (r / 4) + 4 hl + r % 4, MSA row s0 + bn, channel r32. The 16 gate
  // values of a block are loaded (rows clamped to N - 1) before its first store, so their latencies overlap.
  const int d = r32;
#pragma unroll
  for (int bn = 0; bn < 4; bn++) {
    const int s = s0 + bn;
    if (s >= S) continue;  // wave-uniform
    const float* gs = g + (int64_t)s * N * ldg + 32 * h + d;
    float* os = out + (int64_t)s * N * ldo + 32 * h + d;
    float gv[16];
#pragma unroll
    for (int r = 0; r < 16; r++) {
      const int i = i0 + 32 * wave + 8 * (r >> 2) + 4 * hl + (r & 3);
      gv[r] = gs[(int64_t)(i < N ? i : N - 1) * ldg];
    }
#pragma unroll
    for (int r = 0; r < 16; r++) {
      const int i = i0 + 32 * wave + 8 * (r >> 2) + 4 * hl + (r & 3);
      if (i < N) os[(int64_t)i * ldo] = acc[bn][r] * sigmoidf_(gv[r]);
    }
  }
}

}  // namespace

hipError_t launch_opm_split(const float* ab, int64_t ld_ab, const float* mask, void* planes, int S, int N,
                            hipStream_t st) {
  const auto al = [](const void* p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0; };
  const int G = (S + 15) / 16;
  if (S < 1 || N < 1 || G > 65535 || ld_ab < 64 || (int64_t)N * OPM_TOKB > INT32_MAX || !al(planes, 16))
    return hipErrorInvalidValue;
  opm_split_k<<<dim3((unsigned)((N + 1) / 2), (unsigned)G), 256, 0, st>>>(ab, ld_ab, mask,
                                                                           static_cast<__bf16*>(planes), S, N);
  return hipGetLastError();
}

hipError_t launch_opm_outer(const void* planes, const float* num, void* out, int out_dt, int S, int N, int i_base,
                            int n_i, hipStream_t st) {
  const auto al = [](const void* p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0; };
  if (S < 1 || N < 1 || i_base < 0 || n_i < 1 || i_base + n_i > N || (int64_t)N * OPM_TOKB > INT32_MAX ||
      !al(planes, 16))
    return hipErrorInvalidValue;
  const int G = (S + 15) / 16;
  const __bf16* pl = static_cast<const __bf16*>(planes);
  const dim3 grid((unsigned)((N + 3) / 4), (unsigned)((n_i + 3) / 4));
  if (out_dt == DT_F16)
    opm_outer_k<half_t><<<grid, 256, 0, st>>>(pl, num, static_cast<half_t*>(out), G, N, i_base, n_i);
  else
    opm_outer_k<float><<<grid, 256, 0, st>>>(pl, num, static_cast<float*>(out), G, N, i_base, n_i);
  return hipGetLastError();
}

hipError_t launch_pwa_softmax(const float* logits, const float* pm, float inf, float* w, int N, int64_t ldw, int H,
                              hipStream_t st) {
  if (N < 1 || H < 1 || ldw < N || ldw % KS) return hipErrorInvalidValue;
  const int64_t rows = (int64_t)H * N;
  pwa_softmax_k<<<(unsigned)((rows + 3) / 4), 256, 0, st>>>(logits, pm, inf, w, N, ldw, rows);
  return hipGetLastError();
}

int64_t pwa_wsplit_bytes(int N, int64_t ldw, int H) {
  return (int64_t)H * ((N + 31) / 32) * ((ldw / KS + 1) & ~1) * 3 * 1024;
}

hipError_t launch_pwa_wsplit(const float* w, int64_t ldw, void* wp, int N, int H, hipStream_t st) {
  const auto al = [](const void* p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0; };
  if (N < 1 || H < 1 || H > 65535 || ldw < N || ldw % KS || ldw / KS > INT32_MAX || !al(w, 8) || !al(wp, 16))
    return hipErrorInvalidValue;
  const int nib = (N + 31) / 32, njg = (int)((ldw / KS + 1) & ~1);
  pwa_wsplit_k<<<dim3((unsigned)njg, (unsigned)nib, (unsigned)H), 256, 0, st>>>(w, ldw, static_cast<__bf16*>(wp), N,
                                                                                 nib, njg);
  return hipGetLastError();
}

hipError_t launch_pwa_avg(const void* wp, int64_t ldw, const float* v, int64_t ldv, const float* g, int64_t ldg,
                          float* out, int64_t ldo, int S, int N, int H, hipStream_t st) {
  const auto al = [](const void* p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0; };
  if (S < 1 || N < 1 || H < 1 || ldw < N || ldw % KS || ldw / KS > INT32_MAX || ldv % 4 || ldv < 32 * H ||
      ldg < 32 * H || ldo < 32 * H || !al(wp, 16) || !al(v, 16) || S > 4 * 65535 || H > 65535)
    return hipErrorInvalidValue;
  const dim3 grid((unsigned)((N + 127) / 128), (unsigned)((S + 3) / 4), (unsigned)H);
  pwa_avg_k<<<grid, 256, 0, st>>>(static_cast<const __bf16*>(wp), (N + 31) / 32, (int)((ldw / KS + 1) & ~1), v, ldv,
                                  g, ldg, out, ldo, S, N);
  return hipGetLastError();
}

}  // namespace bzpf
