// fp16 flash triangle-attention core on MFMA (v_mfma_f32_32x32x16_f16), head width C = 32.
//
// Work unit: one (head h, row i, 128 queries); 4 waves of 32 queries. The 32 x 32 MFMA form is used throughout: a
// 32-query tile per wave keeps a query's softmax statistics in two lanes (one cross-lane step) and frees registers
// for a fourth wave per SIMD (127 VGPRs).
// The logits are formed transposed, S^T = K Q^T + Cinit, one 32-key x 32-query tile per MFMA pair (A = 32 keys of K
// from LDS, B = the wave's Q fragment, held in registers for the whole row), so lane l owns query l % 32 and 16 keys
// of each 32-key tile (8 (e / 4) + 4 (l / 32) + e % 4 in accumulator element e): a query's softmax statistics live
// in lanes l and l ^ 32 and need one cross-lane step per key block. The MFMA accumulator is initialised with
// tri_bias - m (plus the key-mask bias in blocks that hold a masked key), so the matrix core adds the bias and
// subtracts the running maximum. The maximum is raised lazily and without a per-block maximum: each 32-key tile's
// probabilities are formed against the current maximum, and only when a lane's sum of them exceeds 2^15 (some logit
// above the maximum by more than 15, including an fp16 overflow; a wave-uniform branch) is the tile's maximum taken,
// the accumulators rescaled and the tile's probabilities formed again. The probabilities P^T, rounded to fp16 (at
// most 2^15 once accepted, with the same relative precision as below 1), are already the
// B operand of O^T = V^T P^T for the key order the accumulator gives each lane (keys 4h .. 4h + 3, 8 + 4h .. 8 + 4h
// + 3 of every 16-key slab, h = l / 32); V^T is read from LDS in the same order, so P never leaves registers. The
// softmax denominator is accumulated from the fp16 probabilities with v_dot2_f32_f16 (exact products by one, fp32
// sums). The next key block's K, V^T, bias and mask are loaded into registers while the current block computes;
// the bias arrives in the fragment-ordered layout (tb_offset), four 16-byte loads per lane and block, each of them
// one contiguous 1 KB across the wave (whole cache lines), without passing through LDS.
// Logits are base 2: the projection stores q * log2(e)/sqrt(C) and tri_bias * log2(e); the key-mask bias is
// inf*(m-1)*log2(e). A row whose keys are all masked gets uniform weights over its N keys, which is what the
// reference's rounding gives (every logit rounds to -inf*log2(e); boltz_mlx/kernels.py:579-581). Softmax and
// accumulation are fp32, P is rounded to fp16 for the PV product. Key blocks after the row's last unmasked key
// (trailing padded tokens, however many) are not visited: their probabilities are exactly zero.
// Work units are ordered (h, i, query block) and dealt to the 8 XCDs in contiguous ranges, so the blocks of one
// row share K / V^T in their XCD's L2 and each XCD keeps one head's bias resident.
// Reference behaviour: boltz_mlx/kernels_nax.py:323-558 (f16 flash core), kernels.py:531-600.
#include "bzpf_common.h"
#include "bzpf_kernels.h"

namespace bzpf {

namespace {

constexpr int NXCD = 8;

// fp16 element (low or high half of a 32-bit register) + c in one instruction: v_fma_mix_f32 d = x * 1.0 + c with
// an fp16 source, bit-identical to converting first and adding (one rounding) and half the VALU work.
template <int HI>
__device__ __forceinline__ float half_plus(uint32_t pair, float c) {
  float r;
  if constexpr (HI)
    asm("v_fma_mix_f32 %0, %1, 1.0, %2 op_sel:[1,0,0] op_sel_hi:[1,0,0]" : "=v"(r) : "v"(pair), "v"(c));
  else
    asm("v_fma_mix_f32 %0, %1, 1.0, %2 op_sel_hi:[1,0,0]" : "=v"(r) : "v"(pair), "v"(c));
  return r;
}

typedef _Float16 half2_t __attribute__((ext_vector_type(2)));

// max / sum of a value over the two lanes l and l ^ 32 (the two halves of the wave)
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

template <int C, bool GPRE>
__global__ __launch_bounds__(256, 3) void triattn_core_mfma(const half_t* __restrict__ qkg,
                                                            const half_t* __restrict__ vt,
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
  constexpr float PLIM = 32768.0f;  // lazy rescale: a lane's tile sum above 2^15 (some logit > mref + 15)
  // K and V^T tiles double-buffered: block kb is written to buffer kb & 1 before the one barrier of iteration kb,
  // and that buffer was last read in iteration kb - 2, which every wave finished before the barrier of kb - 1.
  __shared__ LDS_ALIGN half_t Ks[2][BK * LDK];
  __shared__ LDS_ALIGN half_t Vs[2][C * LDV];
  __shared__ LDS_ALIGN float Mb[4][BK];  // per-wave key-mask bias of a block that masks a key
  __shared__ float Vmean[C];

  const int64_t u = (int64_t)(blockIdx.x % NXCD) * per_xcd + blockIdx.x / NXCD;
  if (u >= units) return;  // whole workgroup
  const int nqb = (N + WQ - 1) / WQ;
  const int qb = (int)(u % nqb);
  const int64_t hi = u / nqb;
  const int i = (int)(hi % N);
  const int h = (int)(hi / N);

  const int64_t NN = (int64_t)N * N;
  const int t = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6), l = t & 63;
  const int hl = l >> 5, qi = l & 31;  // lane half, query of the lane within the wave's tile
  const half_t* qp = qkg + ((int64_t)h * NN + (int64_t)i * N) * C;
  const half_t* kp = qkg + ((int64_t)(H + h) * NN + (int64_t)i * N) * C;
  const half_t* gp = qkg + ((int64_t)(2 * H + h) * NN + (int64_t)i * N) * C;
  const half_t* vp = vt + ((int64_t)h * N + i) * C * ldk;
  const float* mrow = mask + (int64_t)i * mask_si;
  const int jq = qb * WQ + 32 * wave + qi;
  // channels of the lane's accumulator (O^T rows) and of its gate / output vectors: 8 q + 4 hl + e, q < 4
  half_t* oq = out + ((int64_t)i * N + jq) * (int64_t)(H * C) + h * C;

  // The row's key extent kend (1 + its last unmasked key; 0 when every key is masked), scanned backwards from the
  // end of the row 256 keys at a time: one step for almost every row. Key blocks after kend are skipped. Once an
  // unmasked key has been seen, a masked key's probability is exactly zero (its bias, about -inf*log2(e), puts it
  // more than 25 below the maximum in base 2 for any logit spread under ~inf, and P is fp16), so skipping changes no
  // bit of the result. A row whose keys are all masked gets uniform weights over its N keys (every logit rounds to
  // the same value in the reference): out = sigmoid(g) * mean_k v[k], no key loop. Both decisions come from the
  // workgroup-wide reduction, never a thread's own flag: the branches hold barriers, and the key loop's MFMAs must
  // run with every lane active.
  __shared__ int kend_w[4];
  int kend = 0;
  for (int base = N - 256;; base -= 256) {  // workgroup-uniform
    const int kq = base + t;  // < N
    const uint64_t b = __ballot(kq >= 0 && mrow[(int64_t)kq * mask_sk] != 0.0f);
    if (l == 0) kend_w[wave] = b ? base + 64 * wave + 64 - __clzll(b) : 0;
    __syncthreads();
    kend = max(max(kend_w[0], kend_w[1]), max(kend_w[2], kend_w[3]));
    __syncthreads();  // kend_w is written again by the next step
    if (kend > 0 || base <= 0) break;
  }
  const bool any_key = kend > 0;
  if (!any_key) {
    {
      const int d = t >> 3, part = t & 7;  // 8 lanes per channel
      float sum = 0.f;
      for (int k = part; k < N; k += 8) sum += (float)vp[(int64_t)d * ldk + k];
#pragma unroll
      for (int o = 1; o < 8; o <<= 1) sum += __shfl_xor(sum, o, 64);
      if (part == 0) Vmean[d] = sum / (float)N;
    }
    __syncthreads();
    if (jq < N) {
#pragma unroll
      for (int q = 0; q < 4; q++) {
        const int d0 = 8 * q + 4 * hl;
        const half4 gv = *reinterpret_cast<const half4*>(gp + (int64_t)jq * C + d0);
        half4 ov;
#pragma unroll
        for (int e = 0; e < 4; e++) ov[e] = (half_t)(Vmean[d0 + e] * sigmoidf_((float)gv[e]));
        *reinterpret_cast<half4*>(oq + d0) = ov;
      }
    }
    return;
  }

  // Q fragments for the two 16-channel slabs: lane (query qi, half hl) holds channels 16 m + 8 hl .. + 7
  half8 qf[2];
  {
    const int jc = jq < N ? jq : N - 1;
#pragma unroll
    for (int m = 0; m < 2; m++) qf[m] = *reinterpret_cast<const half8*>(qp + (int64_t)jc * C + 16 * m + 8 * hl);
  }
  f16x oacc;
#pragma unroll
  for (int e = 0; e < 16; e++) oacc[e] = 0.f;
  float m_run = -INFINITY, lsum = 0.f;
  const float munset = -0.5f * inf * LOG2E;
  // mref: the reference the logits are formed against (0 until a key that is not masked has been seen, then the
  // running maximum); plim: a tile whose probabilities (relative to mref) sum to more than it in some lane raises
  // the maximum. Until the maximum is set plim = -inf (every tile raises it); lanes of the padded queries past N
  // (whose bias rows are never written) have plim = +inf and never ask for a rescale, so the result of a real query
  // never depends on them.
  float mref = 0.0f, plim = jq < N ? -INFINITY : INFINITY;
  const float infl = inf * LOG2E;  // key-mask bias inf * (m - 1) * log2(e) = m * infl - infl
  const half2_t one2 = half2_t{(half_t)1.0f, (half_t)1.0f};

  // staging roles: K rows (64 keys x 32 channels) and V^T rows (32 channels x 64 keys), one 16-byte vector each;
  // every wave loads the raw mask values of the block's 64 keys (lane l: key k0 + l)
  const int skey = t >> 2, sd8 = (t & 3) * 8;
  const int vd = t >> 3, vk8 = (t & 7) * 8;
  if (inf < 1e6f) kend = N;
  const int nblk = (kend + BK - 1) / BK;
  half8 kreg, vreg;
  float mraw;
  // Row-local sources as buffer resources: each lane's offset is fixed and the block offset rides in the scalar
  // offset, so the loads need no address arithmetic; keys past N read as zeros (range-checked).
  constexpr int RSRC_CFG = 0x00020000;  // raw buffer, 32-bit data format
  // (offsets and extents as in bzpf_layout.h, which the host-side layout check evaluates at the launcher's limits)
  const __amdgpu_buffer_rsrc_t krs =
      __builtin_amdgcn_make_buffer_rsrc((void*)kp, 0, (int)core_k_extent(N, C), RSRC_CFG);
  const __amdgpu_buffer_rsrc_t vrs =
      __builtin_amdgcn_make_buffer_rsrc((void*)vp, 0, (int)core_v_extent(ldk, C), RSRC_CFG);
  const int koff = core_k_lane(t, C), voff = core_v_lane(t, ldk);
  // bias fragments (fragment-ordered layout): 32 contiguous values per lane per 32-query tile and 64-key block
  const int njt = (N + 31) / 32, nkb = ldk / 64;
  __amdgpu_buffer_rsrc_t brs;
  {
    int jt = qb * (WQ / 32) + wave;
    if (jt >= njt) jt = njt - 1;
    brs = __builtin_amdgcn_make_buffer_rsrc((void*)(tb + (((int64_t)h * njt + jt) * nkb) * 2048), 0,
                                            (int)core_b_extent(ldk), RSRC_CFG);
  }
  half8 bcur[4];  // bias of keys 32 kt + 8 (e / 4) + 4 hl + e % 4: elements 16 kt + e of the lane's 32
  // mask: lane l reads key kb * 64 + l; only the partial last block clamps (to key N - 1)
  // (as a buffer resource over keys 0 .. N - 1 of the row: keys past N read as 0 and are set to -inf below)
  const __amdgpu_buffer_rsrc_t mrs =
      __builtin_amdgcn_make_buffer_rsrc((void*)mrow, 0, (int)core_m_extent(N, mask_sk), RSRC_CFG);
  const int mvo = core_m_lane(l, mask_sk);
  // loads of block kb (kb < nblk; the loop clamps, so it issues them unconditionally)
  auto prefetch = [&](int kb) {
    kreg = __builtin_bit_cast(half8, __builtin_amdgcn_raw_buffer_load_b128(krs, koff, core_k_block(kb, C), 0));
    vreg = __builtin_bit_cast(half8, __builtin_amdgcn_raw_buffer_load_b128(vrs, voff, core_v_block(kb), 0));
    mraw = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(mrs, mvo, core_m_block(kb, mask_sk), 0));
  };
  auto prefetch_bias = [&](int kb) {
#pragma unroll
    for (int v = 0; v < 4; v++)
      bcur[v] = __builtin_bit_cast(half8, __builtin_amdgcn_raw_buffer_load_b128(brs, core_b_lane(v, l),
                                                                                core_b_block(kb), 0));
  };
  // Issue order pinned to the loop's (K, V^T, mask, then bias): the wait counter merges the prologue and the loop
  // back edge at the loop header, and any other order there turns the first wait of every iteration into a wait
  // for all outstanding loads, prefetches included.
  prefetch(0);
  __builtin_amdgcn_sched_barrier(0);
  prefetch_bias(0);
  __builtin_amdgcn_sched_barrier(0);

  half4 gpre[4];  // GPRE: the output gates, loaded during the last key block
  for (int kb = 0; kb < nblk; kb++) {
    const int k0 = kb * BK, buf = kb & 1;
    if (GPRE && kb == nblk - 1) {
      const int jc = jq < N ? jq : N - 1;
#pragma unroll
      for (int q = 0; q < 4; q++) gpre[q] = *reinterpret_cast<const half4*>(gp + (int64_t)jc * C + 8 * q + 4 * hl);
    }
    half_t* Kb = Ks[buf];
    half_t* Vb = Vs[buf];
    *reinterpret_cast<half8*>(Kb + skey * LDK + sd8) = kreg;
    if (k0 + BK > N) {
#pragma unroll
      for (int e = 0; e < 8; e++)
        if (k0 + vk8 + e >= N) vreg[e] = (half_t)0.0f;
    }
    {
      // keys 8 u .. 8 u + 7 (u = vk8 / 8) go to two 4-key runs: within each 16-key slab, key 8 a + 4 h + e sits at
      // 8 h + 4 a + e, so the 8 keys a lane half multiplies (4 hl .. 4 hl + 3, 8 + 4 hl .. 8 + 4 hl + 3) are one
      // 16-byte read
      const int u = vk8 >> 3;
      half_t* vd0 = Vb + vd * LDV + 16 * (u >> 1) + 4 * (u & 1);
      const u32x4_t vw = __builtin_bit_cast(u32x4_t, vreg);
      *reinterpret_cast<uint2*>(vd0) = uint2{vw[0], vw[1]};
      *reinterpret_cast<uint2*>(vd0 + 8) = uint2{vw[2], vw[3]};
    }
    // key-mask bias of key k0 + l (keys past N: -inf); uniform across waves, so each wave decides by itself
    const float mbias = k0 + l < N ? fmaf(mraw, infl, -infl) : -INFINITY;
    const bool masked = __any(mbias != 0.0f);
    if (masked) Mb[wave][l] = mbias;
    __syncthreads();
    prefetch(kb + 1 < nblk ? kb + 1 : nblk - 1);

    // the maximum is "unset" until a key that is not masked has been seen (a masked logit is about
    // -inf*log2(e)); subtracting such a maximum would cancel catastrophically
    f16x s[2];
#pragma unroll
    for (int kt = 0; kt < 2; kt++) {
      half8 kf[2];
#pragma unroll
      for (int m = 0; m < 2; m++)
        kf[m] = *reinterpret_cast<const half8*>(Kb + (32 * kt + qi) * LDK + 16 * m + 8 * hl);
      f16x c;
      if (masked) {
#pragma unroll
        for (int q = 0; q < 4; q++) {
          const f4 mbv = *reinterpret_cast<const f4*>(&Mb[wave][32 * kt + 8 * q + 4 * hl]);
          const half8 bh = bcur[2 * kt + (q >> 1)];
#pragma unroll
          for (int e = 0; e < 4; e++) c[4 * q + e] = ((float)bh[4 * (q & 1) + e] + mbv[e]) - mref;
        }
      } else {
#pragma unroll
        for (int v = 0; v < 2; v++) {
          const u32x4_t bw = __builtin_bit_cast(u32x4_t, bcur[2 * kt + v]);
#pragma unroll
          for (int w = 0; w < 4; w++) {
            c[8 * v + 2 * w] = half_plus<0>(bw[w], -mref);
            c[8 * v + 2 * w + 1] = half_plus<1>(bw[w], -mref);
          }
        }
      }
      c = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf[0], qf[0], c, 0, 0, 0);
      s[kt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf[1], qf[1], c, 0, 0, 0);
    }
    prefetch_bias(kb + 1 < nblk ? kb + 1 : nblk - 1);  // the bias registers are free once the logits are formed
    float sref = mref;  // s holds logit - sref (a rescale moves it to the new maximum for the block's later tiles)
#pragma unroll
    for (int kt = 0; kt < 2; kt++) {
      // P = 2^(logit - mref) in fp16 for the tile's 32 keys, and the lane's sum of them
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
      // a lane's sum above plim (2^15 once the maximum is set) means some logit exceeds mref by more than 15 (or
      // an fp16 overflow): raise the maximum to the block's remaining tiles, rescale, and form P again
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
        oacc *= corr;
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
        // keys 32 kt + 16 sl + {4 hl .. 4 hl + 3, 8 + 4 hl .. 8 + 4 hl + 3}: accumulator elements 8 sl .. 8 sl + 7
        const half8 vf = *reinterpret_cast<const half8*>(Vb + qi * LDV + 32 * kt + 16 * sl + 8 * hl);
        oacc = __builtin_amdgcn_mfma_f32_32x32x16_f16(vf, pf[sl], oacc, 0, 0, 0);
      }
    }
  }
  // oacc[4 q + e] = O^T[channel 8 q + 4 hl + e][query qi]; the denominator is split over the lane halves
  const float ltot = halves_sum(lsum);
  if (jq >= N) return;
  const float inv = 1.0f / ltot;
#pragma unroll
  for (int q = 0; q < 4; q++) {
    const int d0 = 8 * q + 4 * hl;
    const half4 gv = GPRE ? gpre[q] : *reinterpret_cast<const half4*>(gp + (int64_t)jq * C + d0);
    half4 ov;
#pragma unroll
    for (int e = 0; e < 4; e++) ov[e] = (half_t)(oacc[4 * q + e] * inv * sigmoidf_((float)gv[e]));
    *reinterpret_cast<half4*>(oq + d0) = ov;
  }
}

}  // namespace

hipError_t launch_triattn_core_f16_mfma(const void* qkg, const void* vt, const void* tb, const float* mask,
                                        int64_t mask_si, int64_t mask_sk, float inf, void* out, int64_t N,
                                        int64_t ldk, int H, int C, hipStream_t st) {
  // 32-bit buffer offsets: the mask row (keys 0 .. N - 1 at stride mask_sk floats) and the K / V^T / bias rows
  if (!core_shape_ok(N, ldk, C, mask_sk)) return hipErrorInvalidValue;
  const int64_t units = (int64_t)H * N * ((N + 127) / 128);
  const int64_t per_xcd = (units + NXCD - 1) / NXCD;
  const dim3 grid((unsigned)(per_xcd * NXCD));
  if (N <= 512)
    triattn_core_mfma<32, true><<<grid, 256, 0, st>>>(static_cast<const half_t*>(qkg), static_cast<const half_t*>(vt),
                                                      static_cast<const half_t*>(tb), mask, mask_si, mask_sk, inf,
                                                      static_cast<half_t*>(out), (int)N, (int)ldk, H, units, per_xcd);
  else
    triattn_core_mfma<32, false><<<grid, 256, 0, st>>>(static_cast<const half_t*>(qkg), static_cast<const half_t*>(vt),
                                                       static_cast<const half_t*>(tb), mask, mask_si, mask_sk, inf,
                                                       static_cast<half_t*>(out), (int)N, (int)ldk, H, units, per_xcd);
  return hipGetLastError();
}

}  // namespace bzpf
