// fp16 flash triangle-attention core on MFMA (v_mfma_f32_16x16x32_f16), head width C = 32.
//
// Work unit: one (row i, head h, 64 queries); 4 waves of 16 queries. The logits are formed transposed,
// S^T = K Q^T (A = a 16-key tile of K from LDS, B = the wave's Q fragment held in registers for the whole row), so
// that every lane owns one query (l % 16) and 4 keys of each 16-key tile: the softmax statistics of a query live in
// the 4 lanes l, l^16, l^32, l^48 and need two cross-lane steps per key block. The probabilities P^T are already
// laid out as the B operand of O^T = V^T P^T (V staged transposed in LDS), so P never leaves registers.
// Softmax and accumulation are fp32; the logit order follows the reference: (q.k * scale + mask_bias) + tri_bias
// (boltz_mlx/kernels.py:579-581), so a fully masked row (every logit rounds to -1e9) gives uniform weights.
// Reference behaviour: boltz_mlx/kernels_nax.py:323-558 (f16 flash core), kernels.py:531-600.
#include "bzpf_common.h"
#include "bzpf_kernels.h"

namespace bzpf {

namespace {

typedef _Float16 half2_t __attribute__((ext_vector_type(2)));

template <int C>
__global__ __launch_bounds__(256) void triattn_core_mfma(const half_t* __restrict__ qkvg,
                                                         const half_t* __restrict__ tb,
                                                         const float* __restrict__ mask, int64_t mask_si,
                                                         int64_t mask_sk, float inf, half_t* __restrict__ out,
                                                         int64_t N, int H) {
  static_assert(C == 32, "MFMA core is written for head width 32");
  constexpr int BK = 64;             // keys per LDS stage
  constexpr int LDK = C + 8;         // Ks row pitch (halves)
  constexpr int LDV = BK + 8;        // Vt row pitch (halves)
  __shared__ LDS_ALIGN half_t Ks[BK * LDK];
  __shared__ LDS_ALIGN half_t Vt[C * LDV];
  __shared__ float Mb[BK];

  const int64_t NN = N * N;
  const int64_t i = blockIdx.z;
  const int h = blockIdx.y;
  const int64_t j0 = (int64_t)blockIdx.x * 64;
  const int wave = threadIdx.x >> 6, l = threadIdx.x & 63;
  const int g = l >> 4, qi = l & 15;
  const int64_t jq = j0 + 16 * wave + qi;
  const bool valid = jq < N;
  const int64_t jc = valid ? jq : N - 1;
  const int64_t plane = (int64_t)H * NN * C;  // elements between the q, k, v and g plane groups
  const int64_t rowbase = ((int64_t)h * NN + i * N) * C;
  const half_t* qp = qkvg + rowbase;
  const half_t* kp = qkvg + plane + rowbase;
  const half_t* vp = qkvg + 2 * plane + rowbase;
  const half_t* gp = qkvg + 3 * plane + rowbase;
  const half_t* bp = tb + (int64_t)h * NN + jc * N;  // bias row of this lane's query
  const float scale = 1.0f / sqrtf((float)C);
  constexpr float LOG2E = 1.4426950408889634f;

  const half8 qf = *reinterpret_cast<const half8*>(qp + jc * C + g * 8);
  f4 oacc[2] = {f4{0.f, 0.f, 0.f, 0.f}, f4{0.f, 0.f, 0.f, 0.f}};
  float m = -INFINITY, lsum = 0.f;

  for (int64_t k0 = 0; k0 < N; k0 += BK) {
    __syncthreads();
    {
      const int t = threadIdx.x, key = t >> 2, d8 = (t & 3) * 8;
      const int64_t kk = k0 + key;
      U128 kv = U128{{0u, 0u, 0u, 0u}}, vv = U128{{0u, 0u, 0u, 0u}};
      if (kk < N) {
        kv = *reinterpret_cast<const U128*>(kp + kk * C + d8);
        vv = *reinterpret_cast<const U128*>(vp + kk * C + d8);
      }
      *reinterpret_cast<U128*>(Ks + key * LDK + d8) = kv;
      const half_t* vh = reinterpret_cast<const half_t*>(&vv);
#pragma unroll
      for (int u = 0; u < 8; u++) Vt[(d8 + u) * LDV + key] = vh[u];
      if (t < BK) {
        const int64_t kt = k0 + t;
        Mb[t] = kt < N ? inf * (mask[i * mask_si + kt * mask_sk] - 1.0f) : -INFINITY;
      }
    }
    __syncthreads();
    // S^T tiles: s[t4][e] = logit(query qi, key 16*t4 + 4g + e)
    f4 s[4];
#pragma unroll
    for (int t4 = 0; t4 < 4; t4++) {
      const half8 kf = *reinterpret_cast<const half8*>(Ks + (16 * t4 + qi) * LDK + g * 8);
      s[t4] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf, qf, f4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
    }
    float mloc = -INFINITY;
#pragma unroll
    for (int t4 = 0; t4 < 4; t4++) {
#pragma unroll
      for (int e = 0; e < 4; e++) {
        const int kl = 16 * t4 + 4 * g + e;
        int64_t kk = k0 + kl;
        if (kk >= N) kk = N - 1;  // in-bounds read; the key is excluded by Mb = -inf
        float x = s[t4][e] * scale + Mb[kl];
        x += (float)bp[kk];
        s[t4][e] = x;
        mloc = fmaxf(mloc, x);
      }
    }
    mloc = fmaxf(mloc, __shfl_xor(mloc, 16, 64));
    mloc = fmaxf(mloc, __shfl_xor(mloc, 32, 64));
    const float mn = fmaxf(m, mloc);
    const float corr = exp2f((m - mn) * LOG2E);
    lsum *= corr;
    oacc[0] *= corr;
    oacc[1] *= corr;
    half_t p[4][4];
#pragma unroll
    for (int t4 = 0; t4 < 4; t4++)
#pragma unroll
      for (int e = 0; e < 4; e++) {
        const float pe = exp2f((s[t4][e] - mn) * LOG2E);
        lsum += pe;
        p[t4][e] = (half_t)pe;
      }
    m = mn;
    // O^T += V^T P^T over two 32-key slices
#pragma unroll
    for (int s2 = 0; s2 < 2; s2++) {
      half8 pf;
#pragma unroll
      for (int e = 0; e < 4; e++) {
        pf[e] = p[2 * s2][e];
        pf[4 + e] = p[2 * s2 + 1][e];
      }
#pragma unroll
      for (int dt = 0; dt < 2; dt++) {
        const half_t* vr = Vt + (16 * dt + qi) * LDV + 32 * s2 + 4 * g;
        const half4 lo = *reinterpret_cast<const half4*>(vr);
        const half4 hi = *reinterpret_cast<const half4*>(vr + 16);
        half8 af;
        af[0] = lo[0]; af[1] = lo[1]; af[2] = lo[2]; af[3] = lo[3];
        af[4] = hi[0]; af[5] = hi[1]; af[6] = hi[2]; af[7] = hi[3];
        oacc[dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af, pf, oacc[dt], 0, 0, 0);
      }
    }
  }
  lsum += __shfl_xor(lsum, 16, 64);
  lsum += __shfl_xor(lsum, 32, 64);
  if (!valid) return;
  const float inv = 1.0f / lsum;
  // oacc[dt][e] = O^T[dim 16*dt + 4g + e][query qi]
  const half_t* gq = gp + jq * C;
  half_t* oq = out + (i * N + jq) * (int64_t)(H * C) + h * C;
#pragma unroll
  for (int dt = 0; dt < 2; dt++) {
    const int d0 = 16 * dt + 4 * g;
    const half4 gv = *reinterpret_cast<const half4*>(gq + d0);
    half4 ov;
#pragma unroll
    for (int e = 0; e < 4; e++) ov[e] = (half_t)(oacc[dt][e] * inv * sigmoidf_((float)gv[e]));
    *reinterpret_cast<half4*>(oq + d0) = ov;
  }
}

}  // namespace

hipError_t launch_triattn_core_f16_mfma(const void* qkvg, const void* tb, const float* mask, int64_t mask_si,
                                        int64_t mask_sk, float inf, void* out, int64_t N, int H, int C,
                                        hipStream_t st) {
  if (C != 32) return hipErrorInvalidValue;
  const dim3 grid((unsigned)((N + 63) / 64), (unsigned)H, (unsigned)N);
  triattn_core_mfma<32><<<grid, 256, 0, st>>>(static_cast<const half_t*>(qkvg), static_cast<const half_t*>(tb), mask,
                                              mask_si, mask_sk, inf, static_cast<half_t*>(out), N, H);
  return hipGetLastError();
}

}  // namespace bzpf
