// fp16 sequence attention with pair bias on MFMA (v_mfma_f32_32x32x16_f16), head width HD in {16, 24, 32, 48, 64}
// (24, the s track's 384 / 16, runs its QK product as 32 with zero Q and K dims 24..31):
//   out[j][h*HD + c] = sigmoid(g[j][h*HD + c]) * sum_k softmax_k(q_j.k_k / sqrt(HD) + bias[h][j][k]
//                                                                 + (1 - mask[k]) * -inf) v[k][h*HD + c]
// for the attention of AttentionPairBias (boltz_mlx/layers/attentionv2.py:59-83), the s track's and the diffusion
// transformer's (boltz_mlx/modules/transformersv2.py:218-239).
//
// The structure is the triangle-attention core's (bzpf_triattn_mfma.hip), with the layouts of this path:
// - q, k, v, g are rows of pitch ld_in (the fused q|k|v|g projection), the bias a plain [H][N][N] array and the key
//   mask one fp32 row [N]; grid.y runs over samples (row sets s_in elements apart, mask rows s_mask, output rows
//   s_out), consecutive groups of mult samples sharing one bias (s_bias apart), as the diffusion samples do;
// - a workgroup owns (head h, 32 NW queries), NW = 4 waves of 32 queries (2 when the grid is small); S^T = K Q^T
//   + Cinit over HD / 16 MFMA steps per 32-key tile (Q pre-scaled by log2(e)/sqrt(HD) in the fragments, so logits are base 2), with the accumulator
//   initialised to bias * log2(e) - m (one v_fma_mix_f32 per element from the fp16 bias) plus the key-mask bias in
//   blocks that mask a key;
// - O^T = V^T P^T in 32-channel tiles (ceil(HD / 32) of them; the rows past HD of a partial tile read unused LDS
//   and are never stored); V arrives row-major and is transposed into the LDS V^T tile while it is staged;
// - the lazy rescale, the probability-sum trigger and the padded-query exclusion are the core's. A sequence whose
//   keys are all masked runs without the mask bias (the common -inf shift cancels in the softmax; with the
//   AttentionPairBias inf of 1e6 the reference's fp32 logits keep their differences, unlike the triangle
//   attention's 1e9, which rounds them all to one value).
// Each lane's bias for a 64-key block is eight 8-byte loads (4 consecutive keys each) from its query's row.
#include <type_traits>

#include "bzpf_common.h"
#include "bzpf_kernels.h"

namespace bzpf {

namespace {

typedef _Float16 half2_t __attribute__((ext_vector_type(2)));

// fp16 element (low or high half of a 32-bit register) * m + c in one instruction, fp32 result
template <int HI>
__device__ __forceinline__ float half_fma(uint32_t pair, float m, float c) {
  float r;
  if constexpr (HI)
    asm("v_fma_mix_f32 %0, %1, %2, %3 op_sel:[1,0,0] op_sel_hi:[1,0,0]" : "=v"(r) : "v"(pair), "v"(m), "v"(c));
  else
    asm("v_fma_mix_f32 %0, %1, %2, %3 op_sel_hi:[1,0,0]" : "=v"(r) : "v"(pair), "v"(m), "v"(c));
  return r;
}

__device__ __forceinline__ float halves_max(float v) {
  const unsigned u = __float_as_uint(v);
  const auto a = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  return fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
}
__device__ __forceinline__ float halves_sum(float v) {
  const unsigned u = __float_as_uint(v);
  const auto a = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  return __uint_as_float(a[0]) + __uint_as_float(a[1]);
}

template <int HD, int NW>
__global__ __launch_bounds__(64 * NW, 2) void seq_attn_mfma(const half_t* __restrict__ q, const half_t* __restrict__ k,
                                                        const half_t* __restrict__ v, const half_t* __restrict__ g,
                                                        int64_t ld_in, const half_t* __restrict__ bias,
                                                        const float* __restrict__ mask, float inf,
                                                        half_t* __restrict__ out, int64_t ld_out, int N, int H,
                                                        int S, int64_t s_in, int64_t s_bias, int mult,
                                                        int64_t s_mask, int64_t s_out, int per_xcd) {
  static_assert((HD % 16 == 0 || HD == 24) && HD >= 16 && HD <= 64, "head width 16, 24, 32, 48 or 64");
  constexpr int BK = 64;                   // keys per LDS stage
  constexpr int NTH = 64 * NW;             // threads: NW waves of 32 queries
  constexpr int WQ = 32 * NW;              // queries per workgroup
  constexpr int KS = (HD + 15) / 16;       // QK MFMA steps per 32-key tile (24 runs as 32 with zero dims 24..31)
  constexpr int NT = (HD + 31) / 32;       // 32-channel output tiles
  constexpr int LDK = 16 * KS + 8;         // Ks row pitch (halves)
  constexpr int LDV = BK + 8;              // Vs row pitch (halves)
  constexpr int VPR = HD / 8;              // 16-byte vectors per K / V row
  constexpr int NSTAGE = 2 * BK * VPR;     // staged vectors per block (K then V), a multiple of 64
  constexpr int NV = (NSTAGE + NTH - 1) / NTH;  // per thread
  constexpr float LOG2E = 1.4426950408889634f;
  constexpr float PLIM = 32768.0f;
  // K and V^T tiles double-buffered: block kb is written to buffer kb & 1 before the one barrier of iteration kb,
  // and that buffer was last read in iteration kb - 2, which every wave finished before the barrier of kb - 1.
  __shared__ LDS_ALIGN half_t Ks[2][BK * LDK];
  __shared__ LDS_ALIGN half_t Vs[2][32 * NT * LDV];
  __shared__ LDS_ALIGN float Mb[4][BK];

  // Work units (head, sample, query block), query block fastest, are dealt to the 8 XCDs in contiguous ranges (the
  // dispatcher sends workgroup b to XCD b % 8), so an XCD's units share a few heads' bias planes and their samples'
  // K / V rows in its L2. Sample smp: its own q / k / v / g rows, mask row and output rows; the bias of sample group
  // smp / mult.
  const int nqb = (N + WQ - 1) / WQ;
  const int u = (int)(blockIdx.x % 8) * per_xcd + (int)(blockIdx.x / 8);
  if (u >= nqb * S * H) return;  // whole workgroup
  const int qb = u % nqb;
  const int smp = (u / nqb) % S;
  const int h = u / (nqb * S);
  q += smp * s_in;
  k += smp * s_in;
  v += smp * s_in;
  g += smp * s_in;
  bias += (int64_t)(smp / mult) * s_bias;
  mask += smp * s_mask;
  out += smp * s_out;
  const int t = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6), l = t & 63;
  const int hl = l >> 5, qi = l & 31;
  const int jq = qb * WQ + 32 * wave + qi;
  const int jc = jq < N ? jq : N - 1;
  const half_t* qh = q + h * HD;
  const half_t* kh = k + h * HD;
  const half_t* vh = v + h * HD;
  const half_t* gh = g + h * HD;
  const half_t* bh = bias + (int64_t)h * N * N;

  // A sequence whose keys are all masked adds the same -inf * log2(e) to every logit, which cancels in the softmax
  // (up to the rounding of the reference's fp32 logits near -inf): such a sequence runs without the mask bias.
  bool any_key = __syncthreads_or(l < N && mask[l] != 0.0f) != 0;
  if (!any_key) {
    int found = 0;
    for (int kk = 64 + t; kk < N; kk += NTH) found |= (mask[kk] != 0.0f);
    any_key = __syncthreads_or(found) != 0;
  }

  // Q fragments, scaled to base-2 logits: lane (query qi, half hl) holds dims 16 m + 8 hl .. + 7
  half8 qf[KS];
  {
    const float qs = LOG2E / sqrtf((float)HD);
#pragma unroll
    for (int m = 0; m < KS; m++) {
      const half8 raw = 16 * m + 8 * hl < HD ? *reinterpret_cast<const half8*>(qh + (int64_t)jc * ld_in + 16 * m + 8 * hl)
                                             : half8{0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
      for (int e = 0; e < 8; e++) qf[m][e] = (half_t)((float)raw[e] * qs);
    }
  }
  f16x oacc[NT];
#pragma unroll
  for (int tt = 0; tt < NT; tt++)
#pragma unroll
    for (int e = 0; e < 16; e++) oacc[tt][e] = 0.f;
  float m_run = -INFINITY, lsum = 0.f;
  const float munset = -0.5f * inf * LOG2E;
  float mref = 0.0f, plim = jq < N ? -INFINITY : INFINITY;
  const float infl = inf * LOG2E;
  const float log2e = LOG2E;
  const half2_t one2 = half2_t{(half_t)1.0f, (half_t)1.0f};

  const int nblk = (N + BK - 1) / BK;
  constexpr int RSRC_CFG = 0x00020000;  // raw buffer, 32-bit data format
  // K / V rows (keys past N read as zeros), the bias plane of head h, the mask row
  // (extents as in bzpf_layout.h, which the host-side layout check evaluates at the launcher's limits)
  const __amdgpu_buffer_rsrc_t krs =
      __builtin_amdgcn_make_buffer_rsrc((void*)kh, 0, (int)seqattn_kv_extent(N, ld_in, HD), RSRC_CFG);
  const __amdgpu_buffer_rsrc_t vrs =
      __builtin_amdgcn_make_buffer_rsrc((void*)vh, 0, (int)seqattn_kv_extent(N, ld_in, HD), RSRC_CFG);
  const __amdgpu_buffer_rsrc_t brs =
      __builtin_amdgcn_make_buffer_rsrc((void*)bh, 0, (int)seqattn_bias_extent(N), RSRC_CFG);
  const __amdgpu_buffer_rsrc_t mrs = __builtin_amdgcn_make_buffer_rsrc((void*)mask, 0, N * 4, RSRC_CFG);
  const int boff = (jc * N + 4 * hl) * 2, mvo = l * 4;
  // PF register sets: block kb is loaded PF blocks ahead into set kb % PF (two for 4-wave workgroups, whose VGPR
  // budget holds a second set; one for 2-wave workgroups, which stage twice the vectors per thread)
  constexpr int PF = NW == 4 ? 2 : 1;
  half8 sreg[PF][NV];
  half4 bcur[PF][2][4];  // bias of keys 32 kt + 8 gq + 4 hl + e: accumulator elements 4 gq + e of tile kt
  float mraw[PF];
  // staged vector n of thread t: index e = t + NTH n; e < BK * VPR is K row e / VPR, else V row (e - BK VPR) / VPR
  // The block offset is added to the lane (VGPR) offset, which the buffer range check covers, so keys past N
  // (and the bias of the last query row past its N keys) read as zeros rather than past the allocations.
  auto prefetch = [&](auto si, int kb) {
    constexpr int SI = decltype(si)::value;
    const int blk = (int)((int64_t)kb * BK * ld_in * 2);
#pragma unroll
    for (int n = 0; n < NV; n++) {
      const int e = t + NTH * n;
      if (e >= NSTAGE) break;  // wave-uniform
      const bool isk = e < BK * VPR;
      const int ee = isk ? e : e - BK * VPR;
      const int off = (int)(((int64_t)(ee / VPR) * ld_in + (ee % VPR) * 8) * 2);
      sreg[SI][n] =
          __builtin_bit_cast(half8, __builtin_amdgcn_raw_buffer_load_b128(isk ? krs : vrs, off + blk, 0, 0));
    }
    mraw[SI] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(mrs, mvo + kb * BK * 4, 0, 0));
  };
  auto prefetch_bias = [&](auto si, int kb) {
    constexpr int SI = decltype(si)::value;
    const int bo = boff + kb * BK * 2;
#pragma unroll
    for (int kt = 0; kt < 2; kt++)
#pragma unroll
      for (int gq = 0; gq < 4; gq++)
        bcur[SI][kt][gq] = __builtin_bit_cast(
            half4, __builtin_amdgcn_raw_buffer_load_b64(brs, bo + (32 * kt + 8 * gq) * 2, 0, 0));
  };
  if constexpr (16 * KS > HD) {  // K dims HD .. 16 KS - 1 meet zero Q dims: keep them finite (zero) in both buffers
    for (int r = t; r < 2 * BK; r += NTH)
      *reinterpret_cast<half8*>(Ks[r / BK] + (r % BK) * LDK + HD) = half8{0, 0, 0, 0, 0, 0, 0, 0};
  }
  prefetch(std::integral_constant<int, 0>{}, 0);
  __builtin_amdgcn_sched_barrier(0);
  prefetch_bias(std::integral_constant<int, 0>{}, 0);
  __builtin_amdgcn_sched_barrier(0);
  if constexpr (PF == 2) {
    prefetch(std::integral_constant<int, 1>{}, nblk > 1 ? 1 : 0);
    __builtin_amdgcn_sched_barrier(0);
    prefetch_bias(std::integral_constant<int, 1>{}, nblk > 1 ? 1 : 0);
    __builtin_amdgcn_sched_barrier(0);
  }

  // one key block: stage set kb % PF into LDS buffer kb & 1, load block kb + PF into that set, compute
  auto block = [&](auto si, int kb) {
    constexpr int SI = decltype(si)::value;
    const int k0 = kb * BK, buf = kb & 1;
    half_t* Kb = Ks[buf];
    half_t* Vb = Vs[buf];
#pragma unroll
    for (int n = 0; n < NV; n++) {
      const int e = t + NTH * n;
      if (e >= NSTAGE) break;  // wave-uniform
      if (e < BK * VPR) {  // wave-uniform: BK * VPR is a multiple of 64
        *reinterpret_cast<half8*>(Kb + (e / VPR) * LDK + (e % VPR) * 8) = sreg[SI][n];
      } else {
        const int ee = e - BK * VPR, key = ee / VPR, c0 = (ee % VPR) * 8;
#pragma unroll
        for (int u = 0; u < 8; u++) Vb[(c0 + u) * LDV + key] = sreg[SI][n][u];
      }
    }
    const float mbias = k0 + l < N ? (any_key ? fmaf(mraw[SI], infl, -infl) : 0.0f) : -INFINITY;
    const bool masked = __any(mbias != 0.0f);
    if (masked) Mb[wave][l] = mbias;
    __syncthreads();
    prefetch(si, kb + PF < nblk ? kb + PF : nblk - 1);

    f16x s[2];
#pragma unroll
    for (int kt = 0; kt < 2; kt++) {
      f16x c;
      if (masked) {
#pragma unroll
        for (int gq = 0; gq < 4; gq++) {
          const f4 mbv = *reinterpret_cast<const f4*>(&Mb[wave][32 * kt + 8 * gq + 4 * hl]);
#pragma unroll
          for (int e = 0; e < 4; e++) c[4 * gq + e] = ((float)bcur[SI][kt][gq][e] * LOG2E + mbv[e]) - mref;
        }
      } else {
#pragma unroll
        for (int gq = 0; gq < 4; gq++) {
          const uint2 bw = __builtin_bit_cast(uint2, bcur[SI][kt][gq]);
          c[4 * gq + 0] = half_fma<0>(bw.x, log2e, -mref);
          c[4 * gq + 1] = half_fma<1>(bw.x, log2e, -mref);
          c[4 * gq + 2] = half_fma<0>(bw.y, log2e, -mref);
          c[4 * gq + 3] = half_fma<1>(bw.y, log2e, -mref);
        }
      }
#pragma unroll
      for (int m = 0; m < KS; m++) {
        const half8 kf = *reinterpret_cast<const half8*>(Kb + (32 * kt + qi) * LDK + 16 * m + 8 * hl);
        c = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf, qf[m], c, 0, 0, 0);
      }
      s[kt] = c;
    }
    prefetch_bias(si, kb + PF < nblk ? kb + PF : nblk - 1);
    float sref = mref;
#pragma unroll
    for (int kt = 0; kt < 2; kt++) {
      half8 pf[2];
      float psum = 0.f;
      const auto probs = [&]() {
        psum = 0.f;
#pragma unroll
        for (int sl = 0; sl < 2; sl++) {
#pragma unroll
          for (int e = 0; e < 8; e++) pf[sl][e] = (half_t)__builtin_amdgcn_exp2f(s[kt][8 * sl + e]);
#pragma unroll
          for (int e = 0; e < 8; e += 2)
            psum = __builtin_amdgcn_fdot2(half2_t{pf[sl][e], pf[sl][e + 1]}, one2, psum, false);
        }
      };
      probs();
      if (__any(psum > plim)) {
        float mx = fmaxf(s[kt][0], s[kt][1]);
#pragma unroll
        for (int e = 2; e < 16; e += 2) mx = fmaxf(fmaxf(mx, s[kt][e]), s[kt][e + 1]);
        if (kt == 0) {
#pragma unroll
          for (int e = 0; e < 16; e += 2) mx = fmaxf(fmaxf(mx, s[1][e]), s[1][e + 1]);
        }
        const float mloc = halves_max(mx);
        const float mn = fmaxf(m_run, mloc + sref);
        const float corr = __builtin_amdgcn_exp2f(m_run - mn);
#pragma unroll
        for (int tt = 0; tt < NT; tt++) oacc[tt] *= corr;
        lsum *= corr;
        const float delta = sref - mn;
#pragma unroll
        for (int k2 = kt; k2 < 2; k2++) s[k2] += delta;
        sref = mn;
        m_run = mn;
        const bool unset = m_run <= munset;
        mref = unset ? 0.0f : m_run;
        plim = jq < N ? (unset ? -INFINITY : PLIM) : INFINITY;
        probs();
      }
      lsum += psum;
#pragma unroll
      for (int sl = 0; sl < 2; sl++) {
#pragma unroll
        for (int tt = 0; tt < NT; tt++) {
          // channels 32 tt + qi; keys 32 kt + 16 sl + {4 hl .. 4 hl + 3, 8 + 4 hl .. 8 + 4 hl + 3}
          const half_t* vr = Vb + (32 * tt + qi) * LDV + 32 * kt + 16 * sl + 4 * hl;
          const half4 lo = *reinterpret_cast<const half4*>(vr);
          const half4 hi4 = *reinterpret_cast<const half4*>(vr + 8);
          const half8 vf = half8{lo[0], lo[1], lo[2], lo[3], hi4[0], hi4[1], hi4[2], hi4[3]};
          oacc[tt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vf, pf[sl], oacc[tt], 0, 0, 0);
        }
      }
    }
    };
  for (int kb = 0; kb < nblk; kb += PF) {
    block(std::integral_constant<int, 0>{}, kb);
    if constexpr (PF == 2) {
      if (kb + 1 < nblk) block(std::integral_constant<int, 1>{}, kb + 1);
    }
  }
  // oacc[tt][4 qq + e] = O^T[channel 32 tt + 8 qq + 4 hl + e][query qi]
  const float ltot = halves_sum(lsum);
  if (jq >= N) return;
  const float inv = 1.0f / ltot;
#pragma unroll
  for (int tt = 0; tt < NT; tt++)
#pragma unroll
    for (int qq = 0; qq < 4; qq++) {
      const int d0 = 32 * tt + 8 * qq + 4 * hl;
      if (d0 >= HD) continue;
      const half4 gv = *reinterpret_cast<const half4*>(gh + (int64_t)jq * ld_in + d0);
      half4 ov;
#pragma unroll
      for (int e = 0; e < 4; e++) ov[e] = (half_t)(oacc[tt][4 * qq + e] * inv * sigmoidf_((float)gv[e]));
      *reinterpret_cast<half4*>(out + (int64_t)jq * ld_out + h * HD + d0) = ov;
    }
}

}  // namespace

hipError_t launch_seq_attention_f16_mfma(const void* q, const void* k, const void* v, const void* g, int64_t ld_in,
                                         int64_t s_in, const void* bias, int64_t s_bias, int mult, const float* mask,
                                         int64_t s_mask, float inf, void* out, int64_t ld_out, int64_t s_out,
                                         int S, int64_t N, int H, int hd, hipStream_t st) {
  // 32-bit buffer offsets over a head's K / V rows (block offsets included) and bias plane; 8-byte bias loads need
  // N % 4 == 0, 16-byte row loads ld_in % 8 == 0
  if (!seqattn_shape_ok(N, ld_in) || ld_out % 4 || S < 1 || S > 65535 || mult < 1)
    return hipErrorInvalidValue;
  // 64-query workgroups (2 waves) when 128-query ones would not give two per CU: more of them per CU hide each
  // key block's load latency, and the last query block of a sequence wastes fewer lanes
  const bool small = ((N + 127) / 128) * H * (int64_t)S < 512;
  const int wq = small ? 64 : 128;
  const int64_t units = (N + wq - 1) / wq * (int64_t)S * H, per_xcd = (units + 7) / 8;
  if (units >= (1LL << 31) - 8) return hipErrorInvalidValue;
  const dim3 grid((unsigned)(8 * per_xcd));
#define BZ_SEQ_MFMA(HDV)                                                                                          \
  if (small)                                                                                                     \
    seq_attn_mfma<HDV, 2><<<grid, 128, 0, st>>>(static_cast<const half_t*>(q), static_cast<const half_t*>(k),    \
                                                static_cast<const half_t*>(v), static_cast<const half_t*>(g), ld_in, \
                                                static_cast<const half_t*>(bias), mask, inf,                     \
                                                static_cast<half_t*>(out), ld_out, (int)N, H, S, s_in, s_bias, \
                                                mult, s_mask, s_out, (int)per_xcd);                                                  \
  else                                                                                                           \
    seq_attn_mfma<HDV, 4><<<grid, 256, 0, st>>>(static_cast<const half_t*>(q), static_cast<const half_t*>(k),    \
                                                static_cast<const half_t*>(v), static_cast<const half_t*>(g), ld_in, \
                                                static_cast<const half_t*>(bias), mask, inf,                     \
                                                static_cast<half_t*>(out), ld_out, (int)N, H, S, s_in, s_bias, \
                                                mult, s_mask, s_out, (int)per_xcd)
  switch (hd) {
    case 16: BZ_SEQ_MFMA(16); break;
    case 24: BZ_SEQ_MFMA(24); break;
    case 32: BZ_SEQ_MFMA(32); break;
    case 48: BZ_SEQ_MFMA(48); break;
    case 64: BZ_SEQ_MFMA(64); break;
    default: return hipErrorInvalidValue;
  }
#undef BZ_SEQ_MFMA
  return hipGetLastError();
}

}  // namespace bzpf
