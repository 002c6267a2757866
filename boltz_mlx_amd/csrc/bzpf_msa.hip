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
// Both reductions run on v_mfma_f32_16x16x4f32 (lane l holds A[l % 16][k0 + l / 16] and B[l % 16][k0 + l / 16];
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

// Workgroup tile: rows i0 .. i0 + 127 of head h (A = w[h], row-major with k = j contiguous: As[i][j]) x four MSA
// rows s0 .. s0 + 3 times the head's 32 channels (B = v, Bs[j][s 32 + d], the layout the loads arrive in).
// w rows are zero past N up to ldw (a multiple of 16), so A loads need no column check.
__global__ __launch_bounds__(256, 2) void pwa_avg_k(const float* __restrict__ w, int64_t ldw,
                                                    const float* __restrict__ v, int64_t ldv,
                                                    const float* __restrict__ g, int64_t ldg, float* __restrict__ out,
                                                    int64_t ldo, int S, int N) {
  constexpr int LDA = MBK + 4, LDB = 128 + 16;
  __shared__ LDS_ALIGN float As[2][128 * LDA];
  __shared__ LDS_ALIGN float Bs[2][MBK * LDB];
  const int t = threadIdx.x, wave = t >> 6, l = t & 63;
  const int wm = wave >> 1, wn = wave & 1;
  const int i0 = 128 * (int)blockIdx.x, s0 = 4 * (int)blockIdx.y, h = (int)blockIdx.z;
  const float* wh = w + (int64_t)h * N * ldw;
  f4 ra[2], rb[2];
  auto gload = [&](int stage) {
    const int j0 = stage * MBK;
#pragma unroll
    for (int vv = 0; vv < 2; vv++) {
      const int e = t + 256 * vv;
      const int row = e >> 2, qa = e & 3;  // A: row i0 + row, columns j0 + 4 qa .. + 3
      ra[vv] = i0 + row < N ? *reinterpret_cast<const f4*>(wh + (int64_t)(i0 + row) * ldw + j0 + 4 * qa)
                            : f4{0, 0, 0, 0};
      const int ss = e >> 7, jj = (e >> 3) & 15, qb = e & 7;  // B: MSA row s0 + ss, token j0 + jj, d 4 qb .. + 3
      rb[vv] = (s0 + ss < S && j0 + jj < N)
                   ? *reinterpret_cast<const f4*>(v + ((int64_t)(s0 + ss) * N + j0 + jj) * ldv + 32 * h + 4 * qb)
                   : f4{0, 0, 0, 0};
    }
  };
  auto lstore = [&](int buf) {
#pragma unroll
    for (int vv = 0; vv < 2; vv++) {
      const int e = t + 256 * vv;
      *reinterpret_cast<f4*>(As[buf] + (e >> 2) * LDA + 4 * (e & 3)) = ra[vv];
      *reinterpret_cast<f4*>(Bs[buf] + ((e >> 3) & 15) * LDB + 32 * (e >> 7) + 4 * (e & 7)) = rb[vv];
    }
  };
  f4 acc[4][4];
#pragma unroll
  for (int a = 0; a < 4; a++)
#pragma unroll
    for (int b = 0; b < 4; b++) acc[a][b] = f4{0.f, 0.f, 0.f, 0.f};
  auto compute = [&](int buf) {
    const float* Ab = As[buf] + (64 * wm + (l & 15)) * LDA + (l >> 4);
    const float* Bb = Bs[buf] + (l >> 4) * LDB + 64 * wn + (l & 15);
#pragma unroll
    for (int kk = 0; kk < MBK / 4; kk++) {
      float fa[4], fb[4];
#pragma unroll
      for (int q = 0; q < 4; q++) fa[q] = Ab[16 * q * LDA + 4 * kk];
#pragma unroll
      for (int q = 0; q < 4; q++) fb[q] = Bb[4 * kk * LDB + 16 * q];
#pragma unroll
      for (int a = 0; a < 4; a++)
#pragma unroll
        for (int b = 0; b < 4; b++) acc[a][b] = __builtin_amdgcn_mfma_f32_16x16x4f32(fa[a], fb[b], acc[a][b], 0, 0, 0);
    }
  };
  const int nst = (int)(ldw / MBK);
  gload(0);
  lstore(0);
  __syncthreads();
  for (int st = 0; st < nst; st++) {
    if (st + 1 < nst) gload(st + 1);
    compute(st & 1);
    if (st + 1 < nst) lstore((st + 1) & 1);
    __syncthreads();
  }
  // block (a, b): rows i0 + 64 wm + 16 a + 4 (l / 16) + e, column 64 wn + 16 b + l % 16 = (MSA row, channel d)
#pragma unroll
  for (int b = 0; b < 4; b++) {
    const int col = 64 * wn + 16 * b + (l & 15);
    const int s = s0 + (col >> 5), d = col & 31;
    if (s >= S) continue;
#pragma unroll
    for (int a = 0; a < 4; a++)
#pragma unroll
      for (int e = 0; e < 4; e++) {
        const int i = i0 + 64 * wm + 16 * a + 4 * (l >> 4) + e;
        if (i >= N) continue;
        const int64_t r = (int64_t)s * N + i;
        out[r * ldo + 32 * h + d] = acc[a][b][e] * sigmoidf_(g[r * ldg + 32 * h + d]);
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
