// fp16 flash triangle-attention core on MFMA (v_mfma_f32_16x16x32_f16), head width C = 32.
//
// Work unit: one (head h, row i, 128 queries); 4 waves of 32 queries (two 16-query tiles each). The logits are
// formed transposed, S^T = K Q^T + Cinit (A = a 16-key tile of K from LDS, shared by both query tiles; B = the
// tile's Q fragment, held in registers for the whole row), so every lane owns one query (l % 16) and 4 keys of each
// 16-key tile: a query's softmax statistics live in lanes l, l^16, l^32, l^48 and need two cross-lane steps per key
// block. The MFMA accumulator is initialised with tri_bias - m (plus the key-mask bias in blocks that hold a masked
// key), so the matrix core adds the bias and subtracts the running maximum. The maximum is raised lazily: only when
// a block's logits exceed it by more than 2^8 (a wave-uniform branch) are the accumulators rescaled. The
// probabilities P^T are already laid out as the B operand of O^T = V^T P^T (V^T tiles arrive transposed from the
// projection), so P never leaves registers, and a third MFMA tile whose A operand is a constant row of ones
// accumulates the softmax denominator on the matrix cores. The next key block's K, V^T, bias and mask are loaded
// into registers while the current block computes; the bias arrives in the fragment-ordered layout (tb_offset), two
// 16-byte loads per lane and tile, without passing through LDS.
// Logits are base 2: the projection stores q * log2(e)/sqrt(C) and tri_bias * log2(e); the key-mask bias is
// inf*(m-1)*log2(e). A row whose keys are all masked gets uniform weights over its N keys, which is what the
// reference's rounding gives (every logit rounds to -inf*log2(e); boltz_mlx/kernels.py:579-581). Softmax and
// accumulation are fp32, P is rounded to fp16 for the PV product.
// Work units are ordered (h, i, query block) and dealt to the 8 XCDs in contiguous ranges, so the blocks of one
// row share K / V^T in their XCD's L2 and each XCD keeps one head's bias resident.
// Reference behaviour: boltz_mlx/kernels_nax.py:323-558 (f16 flash core), kernels.py:531-600.
#include "bzpf_common.h"
#include "bzpf_kernels.h"

namespace bzpf {

namespace {

constexpr int NXCD = 8;

template <int C>
__global__ __launch_bounds__(256, 3) void triattn_core_mfma(const half_t* __restrict__ qkg, const half_t* __restrict__ vt,
                                                         const half_t* __restrict__ tb,
                                                         const float* __restrict__ mask, int64_t mask_si,
                                                         int64_t mask_sk, float inf, half_t* __restrict__ out,
                                                         int N, int ldk, int H, int64_t units, int64_t per_xcd) {
  static_assert(C == 32, "MFMA core is written for head width 32");
  constexpr int BK = 64;        // keys per LDS stage
  constexpr int WQ = 128;       // queries per workgroup
  constexpr int LDK = C + 8;    // Ks row pitch (halves)
  constexpr int LDV = BK + 8;   // Vs row pitch (halves)
  constexpr float LOG2E = 1.4426950408889634f;
  constexpr float THRESH = 8.0f;  // lazy rescale threshold (base-2 units)
  __shared__ LDS_ALIGN half_t Ks[BK * LDK];
  __shared__ LDS_ALIGN half_t Vs[C * LDV];
  __shared__ LDS_ALIGN float Mb[BK];
  __shared__ int MaskedFlag;

  const int64_t u = (int64_t)(blockIdx.x % NXCD) * per_xcd + blockIdx.x / NXCD;
  if (u >= units) return;  // whole workgroup
  const int nqb = (N + WQ - 1) / WQ;
  const int qb = (int)(u % nqb);
  const int64_t hi = u / nqb;
  const int i = (int)(hi % N);
  const int h = (int)(hi / N);

  const int64_t NN = (int64_t)N * N;
  const int t = threadIdx.x;
  const int wave = t >> 6, l = t & 63;
  const int g = l >> 4, qi = l & 15;
  const half_t* qp = qkg + ((int64_t)h * NN + (int64_t)i * N) * C;
  const half_t* kp = qkg + ((int64_t)(H + h) * NN + (int64_t)i * N) * C;
  const half_t* gp = qkg + ((int64_t)(2 * H + h) * NN + (int64_t)i * N) * C;
  const half_t* vp = vt + ((int64_t)h * N + i) * C * ldk;
  const float* mrow = mask + (int64_t)i * mask_si;

  // a row with every key masked: uniform weights (all logits equal in the reference's rounding)
  int any_key = 0;
  for (int k = t; k < N; k += 256) any_key |= (mrow[(int64_t)k * mask_sk] != 0.0f);
  const bool row_masked = !__syncthreads_or(any_key);

  int jq[2];
  half8 qf[2];
  f4 oacc[2][3];
  float m[2];
#pragma unroll
  for (int tq = 0; tq < 2; tq++) {
    jq[tq] = qb * WQ + 32 * wave + 16 * tq + qi;
    const int jc = jq[tq] < N ? jq[tq] : N - 1;
    qf[tq] = *reinterpret_cast<const half8*>(qp + (int64_t)jc * C + g * 8);
#pragma unroll
    for (int dt = 0; dt < 3; dt++) oacc[tq][dt] = f4{0.f, 0.f, 0.f, 0.f};
    m[tq] = row_masked ? 0.0f : -INFINITY;
  }
  const float munset = -0.5f * inf * LOG2E;
  half8 ones;
#pragma unroll
  for (int e = 0; e < 8; e++) ones[e] = (half_t)(qi == 0 ? 1.0f : 0.0f);

  // staging roles: K rows (64 keys x 32 channels) and V^T rows (32 channels x 64 keys), one 16-byte vector each
  const int skey = t >> 2, sd8 = (t & 3) * 8;
  const int vd = t >> 3, vk8 = (t & 7) * 8;
  half8 kreg, vreg;
  float mbnext = 0.f;
  // bias fragments (fragment-ordered layout): 16 contiguous values per lane per 16-query tile and 64-key block
  const int njt = (N + 15) / 16, nkb = ldk / 64;
  const half_t* bfp[2];
#pragma unroll
  for (int tq = 0; tq < 2; tq++) {
    int jt = qb * (WQ / 16) + 2 * wave + tq;
    if (jt >= njt) jt = njt - 1;
    bfp[tq] = tb + ((((int64_t)h * njt + jt) * nkb) * 64 + l) * 16;
  }
  half8 bnext[2][2];
  auto prefetch = [&](int k0) {
    int kk = k0 + skey;
    if (kk >= N) kk = N - 1;
    kreg = *reinterpret_cast<const half8*>(kp + (int64_t)kk * C + sd8);
    vreg = *reinterpret_cast<const half8*>(vp + (int64_t)vd * ldk + k0 + vk8);
    if (t < BK) mbnext = k0 + t < N ? inf * (mrow[(int64_t)(k0 + t) * mask_sk] - 1.0f) * LOG2E : -INFINITY;
  };
  auto prefetch_bias = [&](int k0) {
#pragma unroll
    for (int tq = 0; tq < 2; tq++) {
      const half_t* bq = bfp[tq] + (int64_t)(k0 / 64) * 1024;
      bnext[tq][0] = *reinterpret_cast<const half8*>(bq);
      bnext[tq][1] = *reinterpret_cast<const half8*>(bq + 8);
    }
  };
  prefetch(0);
  prefetch_bias(0);

  for (int k0 = 0; k0 < N; k0 += BK) {
    const bool tail = k0 + BK > N;
    __syncthreads();  // the previous block's LDS reads are done
    *reinterpret_cast<half8*>(Ks + skey * LDK + sd8) = kreg;
    if (tail) {
#pragma unroll
      for (int e = 0; e < 8; e++)
        if (k0 + vk8 + e >= N) vreg[e] = (half_t)0.0f;
    }
    *reinterpret_cast<half8*>(Vs + vd * LDV + vk8) = vreg;
    if (t < BK) Mb[t] = mbnext;
    if (wave == 0) {
      const bool any_masked = __any(mbnext != 0.0f);
      if (l == 0) MaskedFlag = any_masked;
    }
    __syncthreads();
    const bool masked = MaskedFlag != 0;
    if (k0 + BK < N) prefetch(k0 + BK);

    half8 kf[4];
#pragma unroll
    for (int t4 = 0; t4 < 4; t4++) kf[t4] = *reinterpret_cast<const half8*>(Ks + (16 * t4 + qi) * LDK + g * 8);
    f4 s[2][4];
    if (row_masked) {
      // uniform weights over keys < N: logit 0 with m = 0
#pragma unroll
      for (int tq = 0; tq < 2; tq++)
#pragma unroll
        for (int t4 = 0; t4 < 4; t4++)
#pragma unroll
          for (int e = 0; e < 4; e++) s[tq][t4][e] = (k0 + 16 * t4 + 4 * g + e < N) ? 0.0f : -INFINITY;
    } else {
      // the maximum is "unset" until a key that is not masked has been seen (a masked logit is about
      // -inf*log2(e)); subtracting such a maximum would cancel catastrophically
      float mref[2];
      bool unset[2];
#pragma unroll
      for (int tq = 0; tq < 2; tq++) {
        unset[tq] = m[tq] <= munset;
        mref[tq] = unset[tq] ? 0.0f : m[tq];
#pragma unroll
        for (int t4 = 0; t4 < 4; t4++) {
          const half8 bh = bnext[tq][t4 >> 1];
          const int o4 = (t4 & 1) * 4;
          const half4 bv = half4{bh[o4], bh[o4 + 1], bh[o4 + 2], bh[o4 + 3]};
          f4 c;
          if (masked) {
            const f4 mbv = *reinterpret_cast<const f4*>(Mb + 16 * t4 + 4 * g);
#pragma unroll
            for (int e = 0; e < 4; e++) c[e] = ((float)bv[e] + mbv[e]) - mref[tq];
          } else {
#pragma unroll
            for (int e = 0; e < 4; e++) c[e] = (float)bv[e] - mref[tq];
          }
          s[tq][t4] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf[t4], qf[tq], c, 0, 0, 0);
        }
      }
      if (k0 + BK < N) prefetch_bias(k0 + BK);  // the bias registers are free once the logits are formed
      float mloc[2];
#pragma unroll
      for (int tq = 0; tq < 2; tq++) {
        float mx = -INFINITY;
#pragma unroll
        for (int t4 = 0; t4 < 4; t4++)
          mx = fmaxf(mx, fmaxf(fmaxf(s[tq][t4][0], s[tq][t4][1]), fmaxf(s[tq][t4][2], s[tq][t4][3])));
        mloc[tq] = xgroups_max(mx);
      }
      // s holds logit - mref; raise the maximum only when the block exceeds it by more than 2^THRESH
      const bool need = unset[0] || unset[1] || mloc[0] > THRESH || mloc[1] > THRESH;
      if (__any(need)) {
#pragma unroll
        for (int tq = 0; tq < 2; tq++) {
          const float mn = fmaxf(m[tq], mloc[tq] + mref[tq]);
          const float corr = __builtin_amdgcn_exp2f(m[tq] - mn);
#pragma unroll
          for (int dt = 0; dt < 3; dt++) oacc[tq][dt] *= corr;
          const float delta = mref[tq] - mn;
#pragma unroll
          for (int t4 = 0; t4 < 4; t4++) s[tq][t4] += delta;
          m[tq] = mn;
        }
      }
    }
    // V^T fragments, read after the logits so that their registers reuse those of the K fragments
    half8 vf[2][2];
#pragma unroll
    for (int s2 = 0; s2 < 2; s2++)
#pragma unroll
      for (int dt = 0; dt < 2; dt++) {
        const half_t* vr = Vs + (16 * dt + qi) * LDV + 32 * s2 + 4 * g;
        const half4 lo = *reinterpret_cast<const half4*>(vr);
        const half4 hi4 = *reinterpret_cast<const half4*>(vr + 16);
        vf[s2][dt] = half8{lo[0], lo[1], lo[2], lo[3], hi4[0], hi4[1], hi4[2], hi4[3]};
      }
#pragma unroll
    for (int tq = 0; tq < 2; tq++)
#pragma unroll
      for (int s2 = 0; s2 < 2; s2++) {
        half8 pf;
#pragma unroll
        for (int e = 0; e < 4; e++) {
          pf[e] = (half_t)__builtin_amdgcn_exp2f(s[tq][2 * s2][e]);
          pf[4 + e] = (half_t)__builtin_amdgcn_exp2f(s[tq][2 * s2 + 1][e]);
        }
        oacc[tq][0] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vf[s2][0], pf, oacc[tq][0], 0, 0, 0);
        oacc[tq][1] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vf[s2][1], pf, oacc[tq][1], 0, 0, 0);
        oacc[tq][2] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ones, pf, oacc[tq][2], 0, 0, 0);
      }
  }
  // oacc[tq][dt][e] = O^T[channel 16*dt + 4g + e][query qi]; the row sum is row 0 of tile 2 (lane qi, e = 0)
#pragma unroll
  for (int tq = 0; tq < 2; tq++) {
    const float lsum = __shfl(oacc[tq][2][0], qi, 64);
    if (jq[tq] >= N) continue;
    const float inv = 1.0f / lsum;
    const half_t* gq = gp + (int64_t)jq[tq] * C;
    half_t* oq = out + ((int64_t)i * N + jq[tq]) * (int64_t)(H * C) + h * C;
#pragma unroll
    for (int dt = 0; dt < 2; dt++) {
      const int d0 = 16 * dt + 4 * g;
      const half4 gv = *reinterpret_cast<const half4*>(gq + d0);
      half4 ov;
#pragma unroll
      for (int e = 0; e < 4; e++) ov[e] = (half_t)(oacc[tq][dt][e] * inv * sigmoidf_((float)gv[e]));
      *reinterpret_cast<half4*>(oq + d0) = ov;
    }
  }
}

}  // namespace

hipError_t launch_triattn_core_f16_mfma(const void* qkg, const void* vt, const void* tb, const float* mask,
                                        int64_t mask_si, int64_t mask_sk, float inf, void* out, int64_t N,
                                        int64_t ldk, int H, int C, hipStream_t st) {
  if (C != 32 || ldk % 64 != 0 || ldk < N || N > 65535) return hipErrorInvalidValue;
  const int64_t units = (int64_t)H * N * ((N + 127) / 128);
  const int64_t per_xcd = (units + NXCD - 1) / NXCD;
  const dim3 grid((unsigned)(per_xcd * NXCD));
  triattn_core_mfma<32><<<grid, 256, 0, st>>>(static_cast<const half_t*>(qkg), static_cast<const half_t*>(vt),
                                              static_cast<const half_t*>(tb), mask, mask_si, mask_sk, inf,
                                              static_cast<half_t*>(out), (int)N, (int)ldk, H, units, per_xcd);
  return hipGetLastError();
}

}  // namespace bzpf
