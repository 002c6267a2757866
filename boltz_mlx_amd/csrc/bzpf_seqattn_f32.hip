// fp32 sequence attention with pair bias on the fp32 matrix cores (v_mfma_f32_32x32x2f32: fp32 products, fp32
// accumulation), head width HD in {16, 24, 32, 48, 64}:
//   out[j][h*HD + c] = sigmoid(g[j][h*HD + c]) * sum_k softmax_k(q_j.k_k / sqrt(HD) + bias[h][j][k]
//                                                                 + (1 - mask[k]) * -inf) v[k][h*HD + c]
// This is the arithmetic of AttentionPairBias in both of the reference's precision modes (boltz_mlx/layers/
// attentionv2.py:50-84: fp32 projections, logits and softmax; in f16 mode the pair bias alone is fp16, so the bias
// type TB is float or half_t).
//
// A workgroup owns (head h, 32 queries) and splits the keys over its NK waves: wave w takes the 32-key tiles
// w, w + NK, ... (grid.y runs over samples, mult consecutive samples sharing one bias, as in the fp16 kernel,
// bzpf_seqattn_mfma.hip). Each wave forms S^T = K Q^T for its tile on the matrix core, in base 2: Q is pre-scaled by
// log2(e)/sqrt(HD) and the accumulators start at log2(e) * (bias + mask term). The MFMA's K = 2 splits the head
// dimension between the two lane halves (half hl takes dims hl*HD/2 .. hl*HD/2 + HD/2 - 1), so lane (key qi, hl)
// reads its K fragment straight from the key's row. In the accumulator lane l holds query l % 32 and the 16 keys
// 8 (r / 4) + 4 hl + r % 4 of the tile (register r); the tile maximum is one permlane32 swap away and the
// probabilities are exact exp2 of the shifted logits. O^T = V^T P^T takes register r of the probabilities as the B
// operand of step r, with V^T read at the same keys from the wave's own LDS copy of the tile's V rows (written and
// read by the one wave in program order, so the loop has no workgroup barrier). The next tile's K, V, bias and mask
// values are loaded while the current tile's softmax and PV product run. At the end the NK partial states
// (running maximum, sum, O^T) are merged through LDS.
// A sequence whose keys are all masked runs without the mask term (a common shift, cancelled by the softmax), as
// the fp16 kernel does.
#include "bzpf_common.h"
#include "bzpf_kernels.h"

namespace bzpf {

namespace {

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

template <typename TB, int HD, int NK>
__global__ __launch_bounds__(64 * NK) void seq_attn_f32_mfma(const float* __restrict__ q, const float* __restrict__ k,
                                                          const float* __restrict__ v, const float* __restrict__ g,
                                                          int64_t ld_in, const TB* __restrict__ bias,
                                                          const float* __restrict__ mask, float inf,
                                                          float* __restrict__ out, int64_t ld_out, int N, int H,
                                                          int64_t s_in, int64_t s_bias, int mult, int64_t s_mask,
                                                          int64_t s_out) {
  static_assert(HD % 8 == 0 && HD >= 16 && HD <= 64, "head width 16, 24, 32, 48 or 64");
  constexpr int HH = HD / 2;          // QK MFMA steps (dims per lane half)
  constexpr int HV = HH / 4;          // 16-byte vectors per lane half of a K / V row
  constexpr int NT = (HD + 31) / 32;  // 32-channel output tiles
  // V tile row pitch: 8 mod 16 floats, so the two lane halves (rows 4 apart) read disjoint bank halves
  constexpr int LDV = 32 * NT + 8;
  constexpr int NSLOT = NT * 16;      // accumulator registers per lane
  constexpr float LOG2E = 1.4426950408889634f;
  constexpr float NEG = -3.0e38f;     // logit of a key past N, running maximum before any key (finite: no inf - inf)
  static_assert(NSLOT * 64 <= 32 * LDV, "a wave's partial O^T fits in its V tile area");
  // per wave: the tile's 32 V rows, after the key loop its partial O^T ([register][lane])
  __shared__ LDS_ALIGN float Vs[NK][32 * LDV];
  __shared__ LDS_ALIGN float Mw[NK][32];  // per wave: the tile's mask terms
  __shared__ LDS_ALIGN float Pm[NK][64], Pl[NK][64];

  {
    const int smp = (int)blockIdx.y;
    q += smp * s_in;
    k += smp * s_in;
    v += smp * s_in;
    g += smp * s_in;
    bias += (int64_t)(smp / mult) * s_bias;
    mask += smp * s_mask;
    out += smp * s_out;
  }
  const int nqt = (N + 31) / 32;
  const int qt = (int)(blockIdx.x % nqt);
  const int h = (int)(blockIdx.x / nqt);
  const int t = threadIdx.x;
  const int w = __builtin_amdgcn_readfirstlane(t >> 6), l = t & 63, hl = l >> 5, qi = l & 31;
  const int jq = 32 * qt + qi;
  const int jc = jq < N ? jq : N - 1;
  const TB* brow = bias + (int64_t)h * N * N + (int64_t)jc * N;
  float* vs = Vs[w];

  int found = 0;
  for (int kk = t; kk < N; kk += 64 * NK) found |= (mask[kk] != 0.0f);
  const bool any_key = __syncthreads_or(found) != 0;
  const float minf = inf * LOG2E;

  // Q fragment of lane (query jc, half hl): dims hl*HH .. hl*HH + HH - 1, scaled to base-2 logits
  float qf[HH];
  {
    const float qs = LOG2E / sqrtf((float)HD);
    const float* qr = q + (int64_t)jc * ld_in + h * HD + hl * HH;
#pragma unroll
    for (int s = 0; s < HH; s += 4) {
      const f4 x = *reinterpret_cast<const f4*>(qr + s);
#pragma unroll
      for (int e = 0; e < 4; e++) qf[s + e] = x[e] * qs;
    }
  }
  if constexpr (32 * NT > HD) {  // V channels past HD meet no stored output: keep them zero (never restaged)
    for (int e = l; e < 32 * (32 * NT - HD); e += 64) vs[(e / (32 * NT - HD)) * LDV + HD + e % (32 * NT - HD)] = 0.f;
  }
  f16x oacc[NT];
#pragma unroll
  for (int tt = 0; tt < NT; tt++)
#pragma unroll
    for (int e = 0; e < 16; e++) oacc[tt][e] = 0.f;
  float m_run = NEG, lsum = 0.f;

  // the registers of one tile: lane (key k0 + qi, half hl)'s K and V row pieces, its 16 bias values, the mask value
  // of key k0 + qi
  f4 kr[HV], vr[HV];
  float br[16], mr;
  auto load = [&](int k0) {
    const int key = k0 + qi;
    const bool in = key < N;
    const int64_t row = (int64_t)(in ? key : N - 1) * ld_in + h * HD + hl * HH;
#pragma unroll
    for (int c = 0; c < HV; c++) {
      kr[c] = in ? *reinterpret_cast<const f4*>(k + row + 4 * c) : f4{0.f, 0.f, 0.f, 0.f};
      vr[c] = in ? *reinterpret_cast<const f4*>(v + row + 4 * c) : f4{0.f, 0.f, 0.f, 0.f};
    }
#pragma unroll
    for (int r = 0; r < 16; r++) {
      const int kk = k0 + 8 * (r >> 2) + 4 * hl + (r & 3);
      br[r] = kk < N ? to_f(brow[kk]) : 0.0f;
    }
    mr = in ? mask[key] : 0.0f;
  };

  const int ntile = nqt;  // 32-key tiles: as many as 32-query tiles
  if (w < ntile) load(32 * w);
  for (int kt = w; kt < ntile; kt += NK) {  // wave-uniform
    const int k0 = 32 * kt;
#pragma unroll
    for (int c = 0; c < HV; c++) *reinterpret_cast<f4*>(vs + qi * LDV + hl * HH + 4 * c) = vr[c];
    if (hl == 0) Mw[w][qi] = k0 + qi < N ? (any_key ? (mr - 1.0f) * minf : 0.0f) : NEG;
    __builtin_amdgcn_wave_barrier();
    f16x s;
#pragma unroll
    for (int a = 0; a < 4; a++) {
      const f4 mb = *reinterpret_cast<const f4*>(&Mw[w][8 * a + 4 * hl]);
#pragma unroll
      for (int e = 0; e < 4; e++) s[4 * a + e] = fmaf(br[4 * a + e], LOG2E, mb[e]);
    }
#pragma unroll
    for (int c = 0; c < HV; c++)
#pragma unroll
      for (int e = 0; e < 4; e++) s = __builtin_amdgcn_mfma_f32_32x32x2f32(kr[c][e], qf[4 * c + e], s, 0, 0, 0);
    if (kt + NK < ntile) load(k0 + 32 * NK);  // the next tile's values arrive during this tile's softmax and PV
    float mx = s[0];
#pragma unroll
    for (int r = 1; r < 16; r++) mx = fmaxf(mx, s[r]);
    const float mn = fmaxf(m_run, halves_max(mx));
    const float corr = __builtin_amdgcn_exp2f(m_run - mn);
    float ps = 0.f;
#pragma unroll
    for (int r = 0; r < 16; r++) {
      s[r] = __builtin_amdgcn_exp2f(s[r] - mn);
      ps += s[r];
    }
    lsum = fmaf(lsum, corr, ps);
    m_run = mn;
#pragma unroll
    for (int tt = 0; tt < NT; tt++) oacc[tt] *= corr;
#pragma unroll
    for (int r = 0; r < 16; r++) {
      const int kl = 8 * (r >> 2) + 4 * hl + (r & 3);
#pragma unroll
      for (int tt = 0; tt < NT; tt++)
        oacc[tt] = __builtin_amdgcn_mfma_f32_32x32x2f32(vs[kl * LDV + 32 * tt + qi], s[r], oacc[tt], 0, 0, 0);
    }
    __builtin_amdgcn_wave_barrier();
  }
  // merge the NK partial states (a wave without a tile holds m = NEG, l = 0, O = 0 and adds nothing); each wave's
  // partial O^T goes to its own V tile area, whose last reads (the wave's own) came before in program order
  lsum = halves_sum(lsum);
  Pm[w][l] = m_run;
  Pl[w][l] = lsum;
#pragma unroll
  for (int tt = 0; tt < NT; tt++)
#pragma unroll
    for (int r = 0; r < 16; r++) vs[(16 * tt + r) * 64 + l] = oacc[tt][r];
  __syncthreads();
  float M = Pm[0][l];
#pragma unroll
  for (int u = 1; u < NK; u++) M = fmaxf(M, Pm[u][l]);
  float wt[NK], L = 0.f;
#pragma unroll
  for (int u = 0; u < NK; u++) {
    wt[u] = __builtin_amdgcn_exp2f(Pm[u][l] - M);
    L = fmaf(wt[u], Pl[u][l], L);
  }
  if (jq >= N) return;
  const float inv = 1.0f / L;
  const float* gr = g + (int64_t)jq * ld_in + h * HD;
  float* orow = out + (int64_t)jq * ld_out + h * HD;
  // wave w writes the registers w, w + NK, ... of the merged O^T
  for (int slot = w; slot < NSLOT; slot += NK) {
    const int tt = slot >> 4, r = slot & 15;
    const int c = 32 * tt + 8 * (r >> 2) + 4 * hl + (r & 3);
    if (c >= HD) continue;
    float o = 0.f;
#pragma unroll
    for (int u = 0; u < NK; u++) o = fmaf(wt[u], Vs[u][slot * 64 + l], o);
    orow[c] = o * inv * sigmoidf_(gr[c]);
  }
}

template <typename TB, int HD>
hipError_t launch_hd(const void* q, const void* k, const void* v, const void* g, int64_t ld_in, int64_t s_in,
                     const void* bias, int64_t s_bias, int mult, const float* mask, int64_t s_mask, float inf,
                     void* out, int64_t ld_out, int64_t s_out, int S, int N, int H, hipStream_t st) {
  // one workgroup per (sample, head, 32 queries); its waves split the keys: 8 when that many workgroups would not
  // give four per CU (and the head fits the register budget of 8-wave workgroups), else 4
  const int64_t wgs = (int64_t)((N + 31) / 32) * H * S;
  const dim3 grid((unsigned)(((N + 31) / 32) * H), (unsigned)S);
  const float* qf = static_cast<const float*>(q);
  const float* kf = static_cast<const float*>(k);
  const float* vf = static_cast<const float*>(v);
  const float* gf = static_cast<const float*>(g);
  const TB* bf = static_cast<const TB*>(bias);
  float* of = static_cast<float*>(out);
  if constexpr (HD <= 32) {
    if (wgs < 1024) {
      seq_attn_f32_mfma<TB, HD, 8><<<grid, 512, 0, st>>>(qf, kf, vf, gf, ld_in, bf, mask, inf, of, ld_out, N, H, s_in,
                                                          s_bias, mult, s_mask, s_out);
      return hipGetLastError();
    }
  }
  seq_attn_f32_mfma<TB, HD, 4><<<grid, 256, 0, st>>>(qf, kf, vf, gf, ld_in, bf, mask, inf, of, ld_out, N, H, s_in,
                                                      s_bias, mult, s_mask, s_out);
  return hipGetLastError();
}

template <typename TB>
hipError_t launch_tb(const void* q, const void* k, const void* v, const void* g, int64_t ld_in, int64_t s_in,
                     const void* bias, int64_t s_bias, int mult, const float* mask, int64_t s_mask, float inf,
                     void* out, int64_t ld_out, int64_t s_out, int S, int N, int H, int hd, hipStream_t st) {
  switch (hd) {
    case 16: return launch_hd<TB, 16>(q, k, v, g, ld_in, s_in, bias, s_bias, mult, mask, s_mask, inf, out, ld_out, s_out, S, N, H, st);
    case 24: return launch_hd<TB, 24>(q, k, v, g, ld_in, s_in, bias, s_bias, mult, mask, s_mask, inf, out, ld_out, s_out, S, N, H, st);
    case 32: return launch_hd<TB, 32>(q, k, v, g, ld_in, s_in, bias, s_bias, mult, mask, s_mask, inf, out, ld_out, s_out, S, N, H, st);
    case 48: return launch_hd<TB, 48>(q, k, v, g, ld_in, s_in, bias, s_bias, mult, mask, s_mask, inf, out, ld_out, s_out, S, N, H, st);
    case 64: return launch_hd<TB, 64>(q, k, v, g, ld_in, s_in, bias, s_bias, mult, mask, s_mask, inf, out, ld_out, s_out, S, N, H, st);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace

// fp32 q / k / v / g / out rows (16-byte aligned bases, pitches and sample strides a multiple of 4 floats), bias of
// type bias_dt; N * N below 2^31 (the bias plane index is 64-bit, the per-row key index 32-bit)
hipError_t launch_seq_attention_f32_mfma(const void* q, const void* k, const void* v, const void* g, int64_t ld_in,
                                         int64_t s_in, const void* bias, int64_t s_bias, int mult, const float* mask,
                                         int64_t s_mask, float inf, void* out, int64_t ld_out, int64_t s_out,
                                         int bias_dt, int S, int64_t N, int H, int hd, hipStream_t st) {
  if (N < 1 || N > 46340 || S < 1 || S > 65535 || mult < 1 || H < 1) return hipErrorInvalidValue;
  return bias_dt == DT_F16
             ? launch_tb<half_t>(q, k, v, g, ld_in, s_in, bias, s_bias, mult, mask, s_mask, inf, out, ld_out, s_out, S,
                                 (int)N, H, hd, st)
             : launch_tb<float>(q, k, v, g, ld_in, s_in, bias, s_bias, mult, mask, s_mask, inf, out, ld_out, s_out, S,
                                (int)N, H, hd, st);
}

}  // namespace bzpf
