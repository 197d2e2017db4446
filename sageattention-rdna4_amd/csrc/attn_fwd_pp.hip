// The main loop as a two-group ping-pong: 8 waves per block, two per SIMD, in two groups of four
// that alternate between the VALU-bound softmax and the MFMA-bound products.
//
// Scheme, layouts and per-score arithmetic are those of attn_fwd.hip (the reference's
// kernels/hip/sk1_t6i.hip:84-299 and sk1_t4a1s.hip): transposed scores S^T = K . Q^T so that a
// lane holds one query, per-key constants as DPP row broadcasts, the exact running max in x units,
// P folded into e4m3 as the P.V operand. What differs is the schedule (and this kernel serves
// head_dim 128 only: at 64 its 8 waves would each stage half a 1 KB request).
//
// Why: per 64-key block a wave spends ~4x longer on its softmax (VALU) than on its MFMAs, and
// the two can only overlap across waves. With two independent waves per SIMD the two tend to hit
// their softmax at the same time and their MFMAs at the same time. Here the two waves sharing a
// SIMD (wave s of group A, wave s of group B) are forced into opposite phases by two barriers per
// block:
//   phase 1 of block j:  A: softmax(j)                 B: P.V(j-1), S^T(j)
//   phase 2 of block j:  A: P.V(j), S^T(j+1)           B: softmax(j)
// so while one wave of a SIMD runs its softmax the other's MFMAs run on the matrix core.
//
// Block: 8 waves x 32 queries = 256 queries of one plane. Wave w = 4g + s (group g, SIMD s)
// owns rows 64s + 32g .. +31 of the block's 256, so both waves of a SIMD share one causal
// diagonal block. K/V^T tiles and per-key constants are staged global -> LDS directly
// (global_load_lds), each of the 8 waves moving one eighth: block j+2's K tile in phase 1 of block
// j, its V^T tile and constants in phase 2, into buffer (j+2) % 3. The only wait is at the end of
// phase 1: it leaves just the K request issued in that phase in flight, so that the K tile of j+1
// (needed in phase 2) and the V^T tile and constants of j+1 have landed.
#include "attn_common.h"
#include "sage_launch.h"

namespace sage {

constexpr int PP_BM = 256;    // queries per block
constexpr int PP_T = 512;     // threads per block
#ifndef PP_NCONV_DEF
#define PP_NCONV_DEF 16
#endif
// int8 Q.K: scores of the next block converted to fp32 at the end of the wave's MFMA phase (which
// has slack) instead of in its softmax phase (issue-bound)
constexpr int PP_NCONV = PP_NCONV_DEF;

template <typename T, bool QK_INT8, bool CAUSAL>
__global__ __launch_bounds__(PP_T) __attribute__((amdgpu_waves_per_eu(2, 2))) void attn_fwd_pp_kernel(
    const T* __restrict__ Q, const u8* __restrict__ K8, const float* __restrict__ KC,
    const u8* __restrict__ V8T, const float* __restrict__ Sfold, T* __restrict__ O, int64_t q_sb,
    int64_t q_sh, int64_t q_sr, int64_t o_sb, int64_t o_sh, int64_t o_sr, int H, int H_kv, int G,
    int N, int Nk, int Nk_pad, int num_qt, int xcd_span, float sm_scale,
    float* __restrict__ LSE, const float* __restrict__ KMEAN,
    const float* __restrict__ VMEAN) {
  __shared__ StageBuf<HD> sB[3];
  using I0 = std::integral_constant<int, 0>;
  using I1 = std::integral_constant<int, 1>;
  using I2 = std::integral_constant<int, 2>;

  // ---- which (plane, q-tile) this block runs: XCD-contiguous planes, longest causal tiles first
  int id = blockIdx.x;
  if (id < xcd_span) id = (id & 7) * (xcd_span >> 3) + (id >> 3);
  const int bh = id / num_qt;
  int qt = id - bh * num_qt;
  if (CAUSAL) qt = num_qt - 1 - qt;
  const int b = bh / H, hd = bh - b * H;
  const int kvp = b * H_kv + hd / G;   // the K/V plane this query plane reads (GQA: G heads share it)

  const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = w >> 2, s = w & 3;
  const int l32 = lane & 31, hh = lane >> 5;
  const int q0 = qt * PP_BM + 64 * s + 32 * g;
  const int qrow = q0 + l32;

  const u8* Kb = K8 + (int64_t)kvp * Nk_pad * HD;
  const u8* Vb = V8T + (int64_t)kvp * HD * Nk_pad;
  const float* KCb = KC + (int64_t)kvp * Nk_pad * 2;   // 128 floats per 64-key block

  const int n_blocks = Nk_pad / BK;
  const int j_end = CAUSAL ? min(n_blocks, (qt * PP_BM + PP_BM - 1) / BK + 1) : n_blocks;
  // blocks this wave computes: 0 .. w_end-1 (the rest of its 2 * j_end barriers it only stages)
  const int w_end = CAUSAL ? min(j_end, (q0 + 31) / BK + 1) : j_end;

  // ---- staging. K: wave w carries rows 8w..8w+7 (lane l: row 8w + l/8, chunk slot l%8 holding
  // logical chunk (l%8) ^ kswz(row)). V^T: rows 16w..16w+15 (lane l: row 16w + l/4, slot l%4
  // holding (l%4) ^ vswz(d)). Constants: waves 0 and 1 carry floats 64w..64w+63 of 128.
  const int krow = 8 * w + (lane >> 3), kpos = lane & 7;
  const uint32_t k_off = (uint32_t)(krow * HD + 16 * (kpos ^ kswz(krow)));
  const int vd = 16 * w + (lane >> 2), vpos = lane & 3;
  const uint32_t v_off = (uint32_t)(vd * Nk_pad + 16 * (vpos ^ vswz(vd)));
  const uint32_t c_off = (uint32_t)(4 * (64 * w + lane));
  const uint32_t lds0 = lds_addr(&sB[0]) + 1024 * w;
  // block j's tiles into buffer p: K (one request per wave), then V^T and constants (one or two).
  // The block offset goes into the per-lane 32-bit offset, so the 64-bit bases stay fixed.
  auto dma_k = [&](int j, int p) {
    dma16(Kb, k_off + (uint32_t)(BK * HD) * (uint32_t)j, lds0 + (uint32_t)p * (uint32_t)sizeof(StageBuf<HD>));
  };
  auto dma_vc = [&](int j, int p) {
    const uint32_t base = lds0 + (uint32_t)p * (uint32_t)sizeof(StageBuf<HD>);
    dma16(Vb, v_off + (uint32_t)BK * (uint32_t)j, base + BK * HD);
    if (w < 2) dma4(KCb, c_off + (uint32_t)(128 * 4) * (uint32_t)j, base + 2 * BK * HD - 768 * w);
  };

  dma_k(0, 0);
  dma_vc(0, 0);
  if (j_end > 1) {
    dma_k(1, 1);
    dma_vc(1, 1);
  }

  // ---- Q: per-row quantization straight into MFMA fragments ----
  QFrag<HD> qf;
  float sq, cq;
  float qmu = 0.0f;   // q . mu for the logsumexp's smooth_k correction (when asked)
  quant_q_row<T, QK_INT8>(Q + b * q_sb + hd * q_sh + (int64_t)qrow * q_sr, qrow < N, hh, sm_scale,
                          qf, sq, cq, (LSE && KMEAN) ? KMEAN + (int64_t)kvp * HD : nullptr, &qmu);
  (void)sq;
  const float Sb = Sfold[kvp];

  f32x16 acc[4];
#pragma unroll
  for (int dt = 0; dt < 4; ++dt)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[dt][r] = 0.0f;
  float m_x = -INFINITY;     // running max of x = (Q8.K8)*SK for this lane's query
  float mc = -INFINITY;      // RN(c_q * m_x), the exp2 shift in use
  float l_i = 0.0f;

  const int krow0 = kappa(0, l32), krow1 = kappa(1, l32);
  const int ksw0 = kswz(krow0), ksw1 = kswz(krow1);
  const int vrow = l32;
  const int vsw = vswz(vrow);

  __builtin_amdgcn_s_waitcnt(0);    // blocks 0 and 1 landed (once per block of queries)
  __syncthreads();

  f32x16 st[2];   // S^T of the block this wave's next softmax works on
  i32x8 pb;       // P of the block this wave's next P.V works on

  auto qk = [&](auto par) {
    constexpr int P = decltype(par)::value;
    qk_block<QK_INT8>(sB[P].k, qf, krow0, krow1, ksw0, ksw1, hh, st);
  };
  float alpha_pend = 1.0f;      // alpha of the block whose P.V comes next
  // P.V of the block whose V^T tile is in buffer p (a compile-time index inside the unrolled
  // loop, a run-time one for the drain after it)
  auto pv_buf = [&](int p) {
    rescale_acc(acc, alpha_pend);
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) {
      const u8* vb = &sB[p].v[(32 * dt + vrow) * BK];
      const i32x4 lo = *(const i32x4*)(vb + 16 * ((2 * hh) ^ vsw));
      const i32x4 hi = *(const i32x4*)(vb + 16 * ((2 * hh + 1) ^ vsw));
      const i32x8 vf = (i32x8){lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
      acc[dt] = mfma_f8(vf, pb, acc[dt]);
    }
  };
  auto pv = [&](auto par) { pv_buf(decltype(par)::value); };
  auto pin_acc = [&]() {
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) asm volatile("" ::"v"(acc[dt]));
  };
  // P.V of block j after the loop, the buffer indexed at run time: one code path, so that the
  // accumulators are not moved between register ranges at a branch join right after the MFMAs
  // (such copies read the MFMA results before the hardware has written them)
  auto pv_rt = [&](int j) {
    pv_buf(j % 3);
    pin_acc();
    mfma_result_fence();
  };
  // softmax of block j on st with its constants, read into registers one phase ahead (during
  // the wave's MFMA phase); the P.V of block j-1 has already been issued
  KeyConsts kcp;
  auto prefetch_consts = [&](auto buf) { kcp = load_key_consts(sB[decltype(buf)::value].s, lane); };
  // The accumulator rescale by alpha is left to the wave's MFMA phase (rescale_pv): a rescale in
  // the softmax phase would hold up all 8 waves at the phase's barrier whenever any one of the 4
  // softmax waves needs it. The softmax phase runs at raised issue priority.
  auto softmax = [&](const int j) {
    __builtin_amdgcn_s_setprio(1);
    const BlockShift sh =
        scores_block<QK_INT8, CAUSAL, QK_INT8 ? PP_NCONV : 0>(st, kcp.sk0, kcp.sk1, j, q0, qrow, Nk,
                                                             hh, cq, m_x, mc);
    probs_block<false>(st, kcp.w0, kcp.w1, cq, sh, l_i, acc, pb);
    alpha_pend = sh.alpha;
    __builtin_amdgcn_s_setprio(0);
  };
  // A phase's products are pinned before its barrier: without the pins the compiler is free to
  // sink MFMAs (which touch no memory) past the barrier into the next phase.
  auto pin_st = [&]() { asm volatile("" ::"v"(st[0]), "v"(st[1])); };
  // (after the phase's last MFMAs: the scheduling barrier keeps the conversions from being hoisted
  // above them, closer to the Q.K MFMAs whose results they read)
  auto preconvert = [&]() {
    if constexpr (QK_INT8) {
      __builtin_amdgcn_sched_barrier(0);
      convert_scores<PP_NCONV>(st);
      pin_st();
    }
  };
  auto pin_pb = [&]() { asm volatile("" ::"v"(pb)); };
  auto end_phase1 = [&](bool more2) {
    __builtin_amdgcn_sched_barrier(0);
    if (more2)
      asm volatile("s_waitcnt vmcnt(1) lgkmcnt(0)\n\ts_barrier" ::: "memory");
    else
      asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
  };
  auto end_phase2 = [&]() {
    __builtin_amdgcn_sched_barrier(0);
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
  };

  // Block j sits in buffer j % 3; block j+2's tiles go to buffer (j+2) % 3, the one block j-1
  // left: its K tile was last read before the previous phase-2 barrier, its V^T tile and
  // constants before this block's phase-1 barrier.
  int j;
  if (g == 0) {
    // group A: phase 1 softmax(j); phase 2 P.V(j), then S^T(j+1) (computed also after the last
    // block, from whatever buffer j+1 holds, and never used: it keeps S^T's live range simple).
    qk(I0{});
    pin_st();
    mfma_result_fence();
    preconvert();
    prefetch_consts(I0{});
    auto blk = [&](const int jj, auto par) {
      constexpr int P = decltype(par)::value;
      constexpr int PN = (P + 1) % 3, PF = (P + 2) % 3;
      const bool more2 = jj + 2 < j_end;
      if (more2) dma_k(jj + 2, PF);
      softmax(jj);
      pin_pb();
      end_phase1(more2);
      if (more2) dma_vc(jj + 2, PF);
      prefetch_consts(std::integral_constant<int, PN>{});   // landed at the barrier above
      // S^T first, P.V after it: the P.V MFMAs then hold this wave's issue until S^T has been
      // written, before the barrier ahead of the softmax that reads it
      qk(std::integral_constant<int, PN>{});
      pin_st();
      __builtin_amdgcn_sched_barrier(0);
      pv(par);
      pin_acc();
      pin_st();
      preconvert();
      end_phase2();
    };
    for (j = 0; j + 3 <= w_end; j += 3) {
      blk(j, I0{});
      blk(j + 1, I1{});
      blk(j + 2, I2{});
    }
    if (j < w_end) {
      blk(j, I0{});
      if (j + 1 < w_end) blk(j + 1, I1{});
    }
    mfma_result_fence();   // the last P.V's results are next read after the loop
  } else {
    // group B: phase 1 P.V(j-1), then S^T(j); phase 2 softmax(j).
    auto blk = [&](const int jj, auto par, auto first) {
      constexpr int P = decltype(par)::value;
      constexpr int PF = (P + 2) % 3;   // block j-1's buffer, block j+2's target
      const bool more2 = jj + 2 < j_end;
      if (more2) dma_k(jj + 2, PF);
      prefetch_consts(par);
      qk(par);
      pin_st();
      __builtin_amdgcn_sched_barrier(0);
      if constexpr (!decltype(first)::value) {
        pv(std::integral_constant<int, PF>{});   // after S^T, as in group A
        pin_acc();
        pin_st();
      } else {
        pin_st();
        mfma_result_fence();   // no P.V behind S^T in the first block
      }
      preconvert();
      end_phase1(more2);
      if (more2) dma_vc(jj + 2, PF);
      softmax(jj);
      pin_pb();
      end_phase2();
    };
    blk(0, I0{}, std::true_type{});
    for (j = 1; j + 3 <= w_end; j += 3) {
      blk(j, I1{}, std::false_type{});
      blk(j + 1, I2{}, std::false_type{});
      blk(j + 2, I0{}, std::false_type{});
    }
    if (j < w_end) {
      blk(j, I1{}, std::false_type{});
      if (j + 1 < w_end) blk(j + 1, I2{}, std::false_type{});
    }
  }
  // Blocks w_end .. j_end-1: stage and keep the barrier count; group B's last P.V runs in the
  // first of them (before block w_end+2's V^T lands in its buffer), or after the loop.
  for (j = w_end; j < j_end; ++j) {
    const bool more2 = j + 2 < j_end;
    const int pf = (j + 2) % 3;
    if (more2) dma_k(j + 2, pf);
    if (g == 1 && j == w_end) pv_rt(j - 1);
    end_phase1(more2);
    if (more2) dma_vc(j + 2, pf);
    end_phase2();
  }
  if (g == 1 && w_end == j_end) pv_rt(j_end - 1);
  // acc is read below only inside the divergent `qrow < N` branch; keep every MFMA out of it
  // (an MFMA under a partial EXEC mask loses the inactive lanes' operand rows).
#pragma unroll
  for (int dt = 0; dt < 4; ++dt) asm volatile("" ::"v"(acc[dt]));
  mfma_result_fence();

  // ---------- epilogue: O = acc * S / (l * 448) (+ V's mean with smooth_v, one fma) ----------
  if (qrow < N) {
    if (LSE && hh == 0) LSE[(int64_t)bh * N + qrow] = row_lse(mc, l_i, sm_scale, qmu);
    const float inv = (l_i > 0.0f) ? __fdiv_rn(Sb, l_i * P_SCALE) : 0.0f;
    T* op = O + b * o_sb + hd * o_sh + (int64_t)qrow * o_sr;
    const float* vmp = VMEAN ? VMEAN + (int64_t)kvp * HD : nullptr;
#pragma unroll
    for (int dt = 0; dt < 4; ++dt)
#pragma unroll
      for (int gg = 0; gg < 4; ++gg) {
        const int d = 32 * dt + 8 * gg + 4 * hh;
        T ov[4];
        if (vmp) {
          const float4 vm = *(const float4*)(vmp + d);
          ov[0] = (T)__builtin_fmaf(acc[dt][4 * gg + 0], inv, vm.x);
          ov[1] = (T)__builtin_fmaf(acc[dt][4 * gg + 1], inv, vm.y);
          ov[2] = (T)__builtin_fmaf(acc[dt][4 * gg + 2], inv, vm.z);
          ov[3] = (T)__builtin_fmaf(acc[dt][4 * gg + 3], inv, vm.w);
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e) ov[e] = (T)(acc[dt][4 * gg + e] * inv);
        }
        uint2 packed;
        __builtin_memcpy(&packed, ov, 8);
        *(uint2*)(op + d) = packed;
      }
  }
}

template <typename T, bool QK_INT8, bool CAUSAL>
static void launch_pp_t(const AttnArgs& a, hipStream_t stream) {
  const int BH = (int)(a.B * a.H);
  const int num_qt = (int)((a.N + PP_BM - 1) / PP_BM);
  const int total = num_qt * BH;
  const int span = (total / 8) * 8;
  hipLaunchKernelGGL((attn_fwd_pp_kernel<T, QK_INT8, CAUSAL>), dim3(total), dim3(PP_T), 0, stream,
                     (const T*)a.q, (const u8*)a.k8, a.kconst, (const u8*)a.v8t, a.s, (T*)a.o,
                     a.q_sb, a.q_sh, a.q_sr, a.o_sb, a.o_sh, a.o_sr, (int)a.H, (int)a.H_kv,
                     (int)(a.H / a.H_kv), (int)a.N, (int)a.N_kv, (int)a.N_kv_pad, num_qt, span,
                     a.sm_scale, a.lse, a.kmean, a.vmean);
}

hipError_t launch_attn_fwd_pp(const AttnArgs& a, hipStream_t stream) {
  if (a.dtype == 1) {
    if (a.causal)
      launch_pp_t<bf16, false, true>(a, stream);
    else
      launch_pp_t<bf16, false, false>(a, stream);
  } else if (a.qk_int8) {
    if (a.causal)
      launch_pp_t<f16, true, true>(a, stream);
    else
      launch_pp_t<f16, true, false>(a, stream);
  } else {
    if (a.causal)
      launch_pp_t<f16, false, true>(a, stream);
    else
      launch_pp_t<f16, false, false>(a, stream);
  }
  return hipGetLastError();
}

}  // namespace sage

