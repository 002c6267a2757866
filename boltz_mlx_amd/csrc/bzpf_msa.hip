// MSA-block pair kernels (fp32 operands and MFMA accumulation, the reference's numerics policy for the reductions
// over MSA rows and tokens):
//   opm_outer   : z[(i - i_base) N + j][c 32 + d] = sum_s mask[s][i] mask[s][j] a[s][i][c] b[s][j][d] / max(num, 1)
//                 with num[i][j] = sum_s mask[s][i] mask[s][j] given (mask^T mask, one small GEMM) and
//                 a | b = ab[s][i][0:32] | ab[s][j][32:64]
//                 (OuterProductMean's outer sum, boltz_mlx/layers/outer_product_mean.py:37-45,
//                 boltz_mlx/kernels_msa.py:292-343), stored fp16 (the proj_o GEMM's operand) or fp32;
//   pwa_softmax : w[h][i][j] = softmax_j(logit[h][i][j] + (1 - pair_mask[i][j]) * -inf), rows padded with zeros
//                 to ldw (boltz_mlx/layers/pair_averaging.py:43-49, kernels_msa.py:461-500);
//   pwa_avg     : out[s][i][h 32 + d] = sigmoid(g[s][i][h 32 + d]) * sum_j w[h][i][j] v[s][j][h 32 + d]
//                 (pair_averaging.py:50-57, kernels_msa.py:620-653).
// The outer sum runs on v_mfma_f32_16x16x4f32 (lane l holds A[l % 16][k0 + l / 16] and B[l % 16][k0 + l / 16];
// the accumulator holds D[4 (l / 16) + e][l % 16]) with a 128 x 128 tile per 256-thread workgroup, 4 waves of
// 64 x 64, K stages of 16 double-buffered in LDS and the next stage's loads in flight during the current one.
#include "bzpf_common.h"
#include "bzpf_kernels.h"

namespace bzpf {

namespace {

constexpr int MBK = 16;  // K (MSA rows s for the outer sum, tokens j for the average) per stage

// ---------------------------------------------------------------- outer product mean
// Workgroup tile: tokens i0 .. i0 + 3 (A rows (i, c)) x j0 .. j0 + 3 (B columns (j, d)). LDS holds each stage
// K-major (As[s][i 32 + c]), the layout the loads arrive in.
template <typename TO>
__global__ __launch_bounds__(256, 2) void opm_outer_k(const float* __restrict__ ab, int64_t ld_ab,
                                                      const float* __restrict__ mask, const float* __restrict__ num,
                                                      TO* __restrict__ out, int S, int N, int i_base, int n_i) {
  constexpr int LD = 128 + 16;
  __shared__ LDS_ALIGN float As[2][MBK * LD];
  __shared__ LDS_ALIGN float Bs[2][MBK * LD];
  const int t = threadIdx.x, wave = t >> 6, l = t & 63;
  const int wm = wave >> 1, wn = wave & 1;
  const int i0 = i_base + 4 * (int)blockIdx.y, j0 = 4 * (int)blockIdx.x;
  const int i_end = min(i_base + n_i, N);
  // vector v of thread t: e = t + 256 v, MSA row s = e / 32, token e / 8 % 4, columns 4 (e % 8) .. + 3
  f4 ra[2], rb[2];
  float ma[2], mb_[2];
  auto gload = [&](int stage) {
#pragma unroll
    for (int v = 0; v < 2; v++) {
      const int e = t + 256 * v, s = stage * MBK + (e >> 5), tk = (e >> 3) & 3, q = e & 7;
      const bool va = s < S && i0 + tk < i_end, vb = s < S && j0 + tk < N;
      ma[v] = va ? mask[(int64_t)s * N + i0 + tk] : 0.0f;
      mb_[v] = vb ? mask[(int64_t)s * N + j0 + tk] : 0.0f;
      ra[v] = va ? *reinterpret_cast<const f4*>(ab + ((int64_t)s * N + i0 + tk) * ld_ab + 4 * q) : f4{0, 0, 0, 0};
      rb[v] = vb ? *reinterpret_cast<const f4*>(ab + ((int64_t)s * N + j0 + tk) * ld_ab + 32 + 4 * q)
                 : f4{0, 0, 0, 0};
    }
  };
  auto lstore = [&](int buf) {
#pragma unroll
    for (int v = 0; v < 2; v++) {
      const int e = t + 256 * v, s = e >> 5, tk = (e >> 3) & 3, q = e & 7;
      *reinterpret_cast<f4*>(As[buf] + s * LD + 32 * tk + 4 * q) = ra[v] * ma[v];
      *reinterpret_cast<f4*>(Bs[buf] + s * LD + 32 * tk + 4 * q) = rb[v] * mb_[v];
    }
  };
  f4 acc[4][4];
#pragma unroll
  for (int a = 0; a < 4; a++)
#pragma unroll
    for (int b = 0; b < 4; b++) acc[a][b] = f4{0.f, 0.f, 0.f, 0.f};
  auto compute = [&](int buf) {
    const float* Ab = As[buf] + (l >> 4) * LD + 64 * wm + (l & 15);
    const float* Bb = Bs[buf] + (l >> 4) * LD + 64 * wn + (l & 15);
#pragma unroll
    for (int kk = 0; kk < MBK / 4; kk++) {
      float fa[4], fb[4];
#pragma unroll
      for (int q = 0; q < 4; q++) fa[q] = Ab[4 * kk * LD + 16 * q];
#pragma unroll
      for (int q = 0; q < 4; q++) fb[q] = Bb[4 * kk * LD + 16 * q];
#pragma unroll
      for (int a = 0; a < 4; a++)
#pragma unroll
        for (int b = 0; b < 4; b++) acc[a][b] = __builtin_amdgcn_mfma_f32_16x16x4f32(fa[a], fb[b], acc[a][b], 0, 0, 0);
    }
  };
  const int nst = (S + MBK - 1) / MBK;
  gload(0);
  lstore(0);
  __syncthreads();
  for (int st = 0; st < nst; st++) {
    if (st + 1 < nst) gload(st + 1);
    compute(st & 1);
    if (st + 1 < nst) lstore((st + 1) & 1);
    __syncthreads();
  }
  // block (a, b) of wave (wm, wn): rows 64 wm + 16 a + 4 (l / 16) + e = (token, c), columns 64 wn + 16 b + l % 16
#pragma unroll
  for (int a = 0; a < 4; a++)
#pragma unroll
    for (int b = 0; b < 4; b++) {
      const int ti = 2 * wm + (a >> 1), tj = 2 * wn + (b >> 1);
      const int i = i0 + ti, j = j0 + tj;
      if (i >= i_end || j >= N) continue;
      const float cnt = fmaxf(num[(int64_t)i * N + j], 1.0f);
      const int d = 16 * (b & 1) + (l & 15);
      TO* op = out + ((int64_t)(i - i_base) * N + j) * 1024 + d;
#pragma unroll
      for (int e = 0; e < 4; e++) {
        const int c = 16 * (a & 1) + 4 * (l >> 4) + e;
        op[c * 32] = (TO)(acc[a][b][e] / cnt);
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

// The average on the bf16 matrix cores at fp32 accuracy. Each fp32 operand value is split exactly into three bf16
// parts, x = x1 + x2 + x3 (x1 the round-to-nearest-even of x, x2 of x - x1, x3 = x - x1 - x2: 8 significant bits
// each, 24 together), and a product is taken as the six part products x_a y_b with a + b <= 4, accumulated in fp32
// by v_mfma_f32_32x32x16_bf16 (exact bf16 products, fp32 sums); the three left out (x2 y3, x3 y2, x3 y3) are below
// 2^-23 of |x y| together. That is the fp32 kernel's accuracy at 6 / 16 of its matrix-core time (the bf16 rate is 16
// times the fp32 one).
// Workgroup tile: rows i0 .. i0 + 127 of head h (A = w[h], k = j) x four MSA rows s0 .. s0 + 3 times the head's 32
// channels (B columns (s, d)); 4 waves of 64 x 64 (2 x 2 blocks of 32 x 32). A stage is 16 tokens j: the loads of
// stage st + 1 are in registers while stage st computes, then split into the parts and stored (LDS double-buffered,
// one barrier per stage). LDS holds each part as its own plane, K-contiguous rows: A[i][j] and B^T[(s, d)][j] (the
// v rows arrive d-contiguous; a thread takes two consecutive tokens of 4 channels and stores each channel's pair
// of parts as one dword).
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

struct Parts3 {
  __bf16 p[3];
};
__device__ __forceinline__ Parts3 split3(float x) {
  Parts3 o;
  o.p[0] = (__bf16)x;
  const float r1 = x - (float)o.p[0];  // exact
  o.p[1] = (__bf16)r1;
  o.p[2] = (__bf16)(r1 - (float)o.p[1]);  // exact: at most 8 significant bits are left
  return o;
}

__global__ __launch_bounds__(256, 2) void pwa_avg_k(const float* __restrict__ w, int64_t ldw,
                                                    const float* __restrict__ v, int64_t ldv,
                                                    const float* __restrict__ g, int64_t ldg, float* __restrict__ out,
                                                    int64_t ldo, int S, int N) {
  constexpr int KS = 16;            // tokens j per stage (one MFMA K-step)
  constexpr int LDP = KS + 8;       // row pitch of a part plane (bf16)
  constexpr int PLANE = 128 * LDP;  // bf16 per plane
  __shared__ LDS_ALIGN __bf16 As[2][3 * PLANE];
  __shared__ LDS_ALIGN __bf16 Bs[2][3 * PLANE];
  const int t = threadIdx.x, wave = t >> 6, l = t & 63, r32 = l & 31, hl = l >> 5;
  const int wm = wave >> 1, wn = wave & 1;
  const int i0 = 128 * (int)blockIdx.x, s0 = 4 * (int)blockIdx.y, h = (int)blockIdx.z;
  const float* wh = w + (int64_t)h * N * ldw;
  // staging roles: A vector vv of thread t is row (t + 256 vv) / 4, tokens 4 ((t + 256 vv) % 4) .. + 3; the B item
  // of thread t is MSA row s0 + t / 64, tokens 2 (t % 8) and 2 (t % 8) + 1, channels 4 ((t / 8) % 8) .. + 3
  const int bp = t & 7, bq = (t >> 3) & 7, bs = t >> 6;
  // two register sets carry the next two stages' values (their loads have two stages of compute to land)
  f4 ra0[2], rb0[2], ra1[2], rb1[2];
  // Loads without conditions: rows past N and MSA rows past S read the last valid ones (their outputs are not
  // stored), and tokens past N read token N - 1's v, which meets w[i][j] = 0 there (w rows are zero past N).
  const int sb = min(s0 + bs, S - 1);
  auto gload = [&](f4 (&ra)[2], f4 (&rb)[2], int stage) {
    const int j0 = stage * KS;
#pragma unroll
    for (int vv = 0; vv < 2; vv++) {
      const int e = t + 256 * vv, row = min(i0 + (e >> 2), N - 1), jq = e & 3;
      ra[vv] = *reinterpret_cast<const f4*>(wh + (int64_t)row * ldw + j0 + 4 * jq);
    }
#pragma unroll
    for (int b = 0; b < 2; b++) {
      const int key = min(j0 + 2 * bp + b, N - 1);
      rb[b] = *reinterpret_cast<const f4*>(v + ((int64_t)sb * N + key) * ldv + 32 * h + 4 * bq);
    }
  };
  auto lstore = [&](const f4 (&ra)[2], const f4 (&rb)[2], int buf) {
#pragma unroll
    for (int vv = 0; vv < 2; vv++) {
      const int e = t + 256 * vv, row = e >> 2, jq = e & 3;
      bf16x4 p1, p2, p3;
#pragma unroll
      for (int q = 0; q < 4; q++) {
        const Parts3 x = split3(ra[vv][q]);
        p1[q] = x.p[0];
        p2[q] = x.p[1];
        p3[q] = x.p[2];
      }
      __bf16* dst = As[buf] + row * LDP + 4 * jq;
      *reinterpret_cast<bf16x4*>(dst) = p1;
      *reinterpret_cast<bf16x4*>(dst + PLANE) = p2;
      *reinterpret_cast<bf16x4*>(dst + 2 * PLANE) = p3;
    }
#pragma unroll
    for (int q = 0; q < 4; q++) {
      const Parts3 x0 = split3(rb[0][q]), x1 = split3(rb[1][q]);
      const bf16x2 p1 = {x0.p[0], x1.p[0]}, p2 = {x0.p[1], x1.p[1]}, p3 = {x0.p[2], x1.p[2]};
      __bf16* dst = Bs[buf] + (32 * bs + 4 * bq + q) * LDP + 2 * bp;
      *reinterpret_cast<bf16x2*>(dst) = p1;
      *reinterpret_cast<bf16x2*>(dst + PLANE) = p2;
      *reinterpret_cast<bf16x2*>(dst + 2 * PLANE) = p3;
    }
  };
  f16x acc[2][2];
#pragma unroll
  for (int a = 0; a < 2; a++)
#pragma unroll
    for (int b = 0; b < 2; b++)
#pragma unroll
      for (int e = 0; e < 16; e++) acc[a][b][e] = 0.0f;
  auto compute = [&](int buf) {
    bf16x8 fa[2][3], fb[2][3];
#pragma unroll
    for (int bm = 0; bm < 2; bm++)
#pragma unroll
      for (int p = 0; p < 3; p++)
        fa[bm][p] = *reinterpret_cast<const bf16x8*>(As[buf] + p * PLANE + (64 * wm + 32 * bm + r32) * LDP + 8 * hl);
#pragma unroll
    for (int bn = 0; bn < 2; bn++)
#pragma unroll
      for (int p = 0; p < 3; p++)
        fb[bn][p] = *reinterpret_cast<const bf16x8*>(Bs[buf] + p * PLANE + (64 * wn + 32 * bn + r32) * LDP + 8 * hl);
#pragma unroll
    for (int bm = 0; bm < 2; bm++)
#pragma unroll
      for (int bn = 0; bn < 2; bn++) {
        // smaller part products first
        f16x c = acc[bm][bn];
        c = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[bm][2], fb[bn][0], c, 0, 0, 0);
        c = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[bm][1], fb[bn][1], c, 0, 0, 0);
        c = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[bm][0], fb[bn][2], c, 0, 0, 0);
        c = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[bm][1], fb[bn][0], c, 0, 0, 0);
        c = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[bm][0], fb[bn][1], c, 0, 0, 0);
        acc[bm][bn] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[bm][0], fb[bn][0], c, 0, 0, 0);
      }
  };
  const int nst = (int)(ldw / KS);
  gload(ra0, rb0, 0);
  lstore(ra0, rb0, 0);
  __syncthreads();
  if (nst > 1) gload(ra0, rb0, 1);
  if (nst > 2) gload(ra1, rb1, 2);
  // stage st computes from buffer st & 1; the stores of stage st + 1 go to the other buffer, whose last reader (stage
  // st - 1) every wave finished before the previous barrier
  for (int st = 0; st < nst; st += 2) {
    compute(0);
    if (st + 1 < nst) lstore(ra0, rb0, 1);
    __syncthreads();
    if (st + 3 < nst) gload(ra0, rb0, st + 3);
    if (st + 1 < nst) {
      compute(1);
      if (st + 2 < nst) lstore(ra1, rb1, 0);
      __syncthreads();
      if (st + 4 < nst) gload(ra1, rb1, st + 4);
    }
  }
  // block (bm, bn) register r: row i0 + 64 wm + 32 bm + 8 (r / 4) + 4 hl + r % 4, column 64 wn + 32 bn + r32 =
  // (MSA row, channel d). All 32 gate values of a column are loaded (rows clamped to N - 1) before any is used, so
  // their latencies overlap instead of following one another.
#pragma unroll
  for (int bn = 0; bn < 2; bn++) {
    const int col = 64 * wn + 32 * bn + r32;
    const int s = s0 + (col >> 5), d = col & 31;
    if (s >= S) continue;  // wave-uniform
    const float* gs = g + (int64_t)s * N * ldg + 32 * h + d;
    float* os = out + (int64_t)s * N * ldo + 32 * h + d;
    float gv[2][16];
#pragma unroll
    for (int bm = 0; bm < 2; bm++)
#pragma unroll
      for (int r = 0; r < 16; r++) {
        const int i = i0 + 64 * wm + 32 * bm + 8 * (r >> 2) + 4 * hl + (r & 3);
        gv[bm][r] = gs[(int64_t)(i < N ? i : N - 1) * ldg];
      }
#pragma unroll
    for (int bm = 0; bm < 2; bm++)
#pragma unroll
      for (int r = 0; r < 16; r++) {
        const int i = i0 + 64 * wm + 32 * bm + 8 * (r >> 2) + 4 * hl + (r & 3);
        if (i < N) os[(int64_t)i * ldo] = acc[bm][bn][r] * sigmoidf_(gv[bm][r]);
      }
  }
}

}  // namespace

hipError_t launch_opm_outer(const float* ab, int64_t ld_ab, const float* mask, const float* num, void* out,
                            int out_dt, int S, int N, int i_base, int n_i, hipStream_t st) {
  const auto al = [](const void* p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0; };
  if (S < 1 || N < 1 || i_base < 0 || n_i < 1 || i_base + n_i > N || ld_ab < 64 || ld_ab % 4 || !al(ab, 16))
    return hipErrorInvalidValue;
  const dim3 grid((unsigned)((N + 3) / 4), (unsigned)((n_i + 3) / 4));
  if (out_dt == DT_F16)
    opm_outer_k<half_t><<<grid, 256, 0, st>>>(ab, ld_ab, mask, num, static_cast<half_t*>(out), S, N, i_base, n_i);
  else
    opm_outer_k<float><<<grid, 256, 0, st>>>(ab, ld_ab, mask, num, static_cast<float*>(out), S, N, i_base, n_i);
  return hipGetLastError();
}

hipError_t launch_pwa_softmax(const float* logits, const float* pm, float inf, float* w, int N, int64_t ldw, int H,
                              hipStream_t st) {
  if (N < 1 || H < 1 || ldw < N || ldw % MBK) return hipErrorInvalidValue;
  const int64_t rows = (int64_t)H * N;
  pwa_softmax_k<<<(unsigned)((rows + 3) / 4), 256, 0, st>>>(logits, pm, inf, w, N, ldw, rows);
  return hipGetLastError();
}

hipError_t launch_pwa_avg(const float* w, int64_t ldw, const float* v, int64_t ldv, const float* g, int64_t ldg,
                          float* out, int64_t ldo, int S, int N, int H, hipStream_t st) {
  const auto al = [](const void* p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0; };
  if (S < 1 || N < 1 || H < 1 || ldw < N || ldw % MBK || ldv % 4 || ldv < 32 * H || ldg < 32 * H ||
      ldo < 32 * H || !al(w, 16) || !al(v, 16) || S > 4 * 65535 || H > 65535)
    return hipErrorInvalidValue;
  const dim3 grid((unsigned)((N + 127) / 128), (unsigned)((S + 3) / 4), (unsigned)H);
  pwa_avg_k<<<grid, 256, 0, st>>>(w, ldw, v, ldv, g, ldg, out, ldo, S, N);
  return hipGetLastError();
}

}  // namespace bzpf
