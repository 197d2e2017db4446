// The quantized flash-attention main loop on gfx950 (CDNA4, wave64 MFMA).
//
// Scheme (the reference's, kernels/hip/sk1_t6i.hip:84-299 and sk1_t4a1s.hip): Q is quantized per
// row inside the kernel (int8 for fp16 inputs, e4m3 for bf16), K8/SK/V8T/SV'/S come from the
// prologue. Per 64-key block: scores s = c_q * SK * (Q8.K8), one running-max update, p =
// exp2(s - m), l += sum p, p8 = e4m3(p * SV' * 448), acc = acc * alpha + p8 . V8; the epilogue
// writes acc * S / (l * 448).
//
// MI355X design:
// * Block = 4 waves x 32 queries (BM = 128). Each wave owns one 32-query tile and computes the
//   TRANSPOSED score tile S^T = K . Q^T with v_mfma_i32_32x32x32_i8 (int8 Q.K) or
//   v_mfma_scale_f32_32x32x64_f8f6f4 (e4m3 Q.K, unit scales). In a 32x32 accumulator lane
//   (q = lane%32, h = lane/32) holds column q -- one query -- so the softmax statistics are per
//   lane, and the accumulator IS the P^T operand of the P.V MFMA (O^T = V^T . P^T) without any
//   LDS round trip or lane shuffle.
// * The K rows fed to the S^T MFMA are permuted so that lane half h receives keys 32h .. 32h+31 of
//   the block in register order; V8T's 32 contiguous bytes per (d, h) are then exactly the V^T
//   operand. (Which K row occupies which MFMA row is free: the reduction is over d.)
// * The softmax is the VALU bottleneck (the MFMA work per score is 256 MACs = 1/16 clock per CU;
//   the VALU runs 64 lanes per clock per CU), so it is written for the fewest VALU instructions per
//   score: x = fp32(Q8.K8) * SK, with SK a DPP row broadcast folded into the multiply (no LDS read
//   per score); the running max is kept in x units per query, so the exp2 argument c_q*x - mc is
//   one fma; p*RN(SV'*448) is another DPP-broadcast multiply. Per score: cvt (int8 only), mul,
//   max3/2, fma, exp2, add, mul, cvt_pk/2.
// * Staging: K, V^T and the per-key constants go global -> LDS directly (global_load_lds), two
//   blocks ahead into three LDS buffers; the DMAs are written as asm so that the loop's own
//   s_waitcnt retires exactly the requests the next block needs, then one barrier per block.
//   K rows use an XOR swizzle of their 16-byte chunks, V^T rows another, so the MFMA operand reads
//   are bank-conflict free.
// * Head dimension D = 128 or 64 (a template parameter): D/32 int8 (D/64 e4m3) Q.K MFMAs per
//   32-key tile, D/32 output tiles, D-byte K rows. Occupancy: 3 waves per SIMD at D = 128, 4 at 64.
// * Grouped K/V heads and a key length of their own: a block of query plane bh reads K/V plane
//   b*H_kv + h/(H/H_kv); keys are bounded and masked by N_kv, queries by N.
// * Causal: blocks past the CTA's diagonal are never visited, a wave skips blocks past its own
//   diagonal, and masks are applied only on diagonal blocks. The grid is a 1-D list of (plane,
//   q-tile) pairs, remapped so that each XCD (workgroup id mod 8) runs a contiguous range of
//   planes (K/V of a plane stay in that XCD's L2), longest causal tiles first.
#include "attn_common.h"
#include "sage_launch.h"

namespace sage {

template <typename T, bool QK_INT8, bool CAUSAL, int D>
__global__ __launch_bounds__(AT) __attribute__((amdgpu_waves_per_eu(attn_waves(D), attn_waves(D)))) void attn_fwd_kernel(
    const T* __restrict__ Q, const u8* __restrict__ K8, const float* __restrict__ KC,
    const u8* __restrict__ V8T, const float* __restrict__ Sfold,
    T* __restrict__ O, int64_t q_sb, int64_t q_sh, int64_t q_sr, int64_t o_sb, int64_t o_sh,
    int64_t o_sr, int H, int H_kv, int G, int N, int Nk, int Nk_pad, int num_qt, int xcd_span,
    float sm_scale, float* __restrict__ LSE, const float* __restrict__ KMEAN,
    const float* __restrict__ VMEAN) {
  // Three staging buffers (K tile, V^T tile, per-key constants), declared as separate objects:
  // with the buffer chosen at compile time the compiler can tell a DMA into one buffer from reads
  // of another, and waits for a DMA only where its own buffer is read. (Its wait bookkeeping
  // tells apart a handful of DMA targets, so there are three objects, not nine.)
  __shared__ StageBuf<D> sB0;
  __shared__ StageBuf<D> sB1;
  __shared__ StageBuf<D> sB2;
  // q . mu of each query row, for the logsumexp's smooth_k correction: parked here rather than
  // in a register that would live (and spill) across the whole loop
  __shared__ float s_qmu[BM];
  constexpr int NDT = D / 32;   // 32-channel output tiles per wave
  constexpr int NKV = D / 64;   // 1 KB K and V^T requests per wave and block (each)

  // ---- which (plane, q-tile) this block runs ----
  int id = blockIdx.x;
  if (id < xcd_span) id = (id & 7) * (xcd_span >> 3) + (id >> 3);
  const int bh = id / num_qt;
  int qt = id - bh * num_qt;
  if (CAUSAL) qt = num_qt - 1 - qt;
  const int b = bh / H, hd = bh - b * H;
  const int kvp = b * H_kv + hd / G;   // the K/V plane this query plane reads (GQA: G heads share it)

  // w is wave-uniform; readfirstlane tells the compiler so, which turns every per-wave decision
  // (causal block skipping) into a scalar branch rather than an EXEC mask.
  const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l32 = lane & 31, hh = lane >> 5;
  const int q0 = qt * BM + w * 32;
  const int qrow = q0 + l32;

  const u8* Kb = K8 + (int64_t)kvp * Nk_pad * D;
  const u8* Vb = V8T + (int64_t)kvp * D * Nk_pad;
  const float* KCb = KC + (int64_t)kvp * Nk_pad * 2;   // 128 floats per 64-key block

  const int n_blocks = Nk_pad / BK;
  const int j_end = CAUSAL ? min(n_blocks, (qt * BM + BM - 1) / BK + 1) : n_blocks;
  const int w_end = CAUSAL ? min(j_end, (q0 + 31) / BK + 1) : j_end;

  // ---- staging: global -> LDS directly (global_load_lds), two blocks ahead into three LDS
  // buffers. Block j+2 is requested at the top of block j, and the wait at the bottom of block j
  // covers only block j+1's requests, so a tile has two blocks of compute to arrive (a plane's K/V
  // exceed an XCD's L2: many requests go to the next cache level). Per block every wave issues
  // exactly 2*NKV + 1 requests (five for D = 128, three for D = 64): NKV KB of K, NKV KB of V^T
  // and 256 bytes of the per-key constants.
  //   K:   request I = NKV*w + i (16 B/lane) carries the 1024/D rows (1024/D)*I ..; lane l lands
  //        at byte 16*l of that KB, i.e. row (1024/D)*I + l/(D/16), chunk slot l%(D/16), which
  //        holds logical chunk slot ^ kswz(row).
  //   V^T: request I carries rows d = 16I..16I+15; lane l -> row 16I + l/4, slot l%4 holding
  //        logical chunk (l%4) ^ vswz(d).
  //   KC:  waves 0 and 1 carry floats 64w..64w+63 of the block's 128 (4 B/lane); waves 2 and 3
  //        repeat them into the tile's pad.
  uint32_t k_off[NKV], v_off[NKV];
#pragma unroll
  for (int i = 0; i < NKV; ++i) {
    const int I = NKV * w + i;
    const int krow = (1024 / D) * I + lane / (D / 16), kpos = lane % (D / 16);
    k_off[i] = (uint32_t)(krow * D + 16 * (kpos ^ kswz<D>(krow)));
    const int d = 16 * I + (lane >> 2), vpos = lane & 3;
    v_off[i] = (uint32_t)(d * Nk_pad + 16 * (vpos ^ vswz(d)));
  }
  const uint32_t c_off = (uint32_t)(4 * (64 * (w & 1) + lane));
  const uint32_t c_dst = (uint32_t)(256 * w);
  auto dma = [&](int j, StageBuf<D>& buf) {
    const u8* kblk = Kb + (size_t)(BK * D) * (uint32_t)j;
    const u8* vblk = Vb + (size_t)BK * (uint32_t)j;
    const u8* cblk = (const u8*)KCb + (size_t)(128 * 4) * (uint32_t)j;
    const uint32_t kl = lds_addr(buf.k) + 1024 * NKV * w, vl = lds_addr(buf.v) + 1024 * NKV * w;
#pragma unroll
    for (int i = 0; i < NKV; ++i) dma16(kblk, k_off[i], kl + 1024 * i);
#pragma unroll
    for (int i = 0; i < NKV; ++i) dma16(vblk, v_off[i], vl + 1024 * i);
    dma4(cblk, c_off, lds_addr(&buf.s) + c_dst);
  };

  // Blocks 0 and 1 are requested before the Q quantization so they overlap it.
  dma(0, sB0);
  if (j_end > 1) dma(1, sB1);

  // ---- Q: per-row quantization straight into MFMA fragments ----
  QFrag<D> qf;
  float sq, cq;
  float qmu = 0.0f;   // q . mu for the logsumexp's smooth_k correction (when asked)
  quant_q_row<T, QK_INT8, D>(Q + b * q_sb + hd * q_sh + (int64_t)qrow * q_sr, qrow < N, hh,
                             sm_scale, qf, sq, cq,
                             (LSE && KMEAN) ? KMEAN + (int64_t)kvp * D : nullptr, &qmu);
  (void)sq;
  if (LSE && hh == 0) s_qmu[32 * w + l32] = qmu;
  const float Sb = Sfold[kvp];

  f32x16 acc[NDT];
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[dt][r] = 0.0f;
  float m_x = -INFINITY;     // running max of x = (Q8.K8)*SK for this lane's query
  float mc = -INFINITY;      // RN(c_q * m_x), the exp2 shift in use
  float l_i = 0.0f;

  const int krow0 = kappa(0, l32), krow1 = kappa(1, l32);
  const int ksw0 = kswz<D>(krow0), ksw1 = kswz<D>(krow1);
  const int vrow = l32;               // + 32 dt
  const int vsw = vswz(vrow);         // vswz(32dt + r) == vswz(r)

  __builtin_amdgcn_s_waitcnt(0);    // blocks 0 and 1 landed (once per block of queries)
  __syncthreads();

  // One 64-key block j, whose tiles are in buffer P = j % 3 (chosen at compile time, so that the
  // compiler can tell the requests in flight to other buffers from this block's reads). At the
  // top: request block j+2 into buffer (P+2) % 3, which block j-1 read and every wave has
  // finished with (barrier). At the bottom: wait until this wave's requests for block j+1 have
  // landed (2*NKV + 1 requests per block, in order: vmcnt(2*NKV + 1) leaves just block j+2's),
  // then barrier.
  // The barrier is written as asm with a memory clobber: a workgroup fence would also wait for
  // block j+2's requests.
  auto block = [&](const int j, auto par) {
    constexpr int P = decltype(par)::value;
    StageBuf<D>& bcur = P == 0 ? sB0 : (P == 1 ? sB1 : sB2);
    StageBuf<D>& bnew = P == 0 ? sB2 : (P == 1 ? sB0 : sB1);
    const u8* const kcur = bcur.k;
    const u8* const vcur = bcur.v;
    const ScaleTile& sc = bcur.s;
    const bool more2 = j + 2 < j_end;
    if (more2) dma(j + 2, bnew);

    if (!CAUSAL || j < w_end) {
      const KeyConsts kc = load_key_consts(sc, lane);
      f32x16 st[2];
      qk_block<QK_INT8, D>(kcur, qf, krow0, krow1, ksw0, ksw1, hh, st);
      // the softmax reads S^T right away: wait out the MFMA's duration first (the compiler's
      // own padding after these MFMAs is shorter than what the hardware was measured to need)
      keep_live(st[0]);
      keep_live(st[1]);
      qk_result_fence<QK_INT8>();
      i32x8 pb;
      softmax_block<QK_INT8, CAUSAL>(st, kc, j, q0, qrow, Nk, hh, cq, m_x, mc, l_i, acc, pb);

      // ---------- O^T += V^T . P^T ----------
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt) {
        const u8* vb = &vcur[(32 * dt + vrow) * BK];
        const i32x4 lo = *(const i32x4*)(vb + 16 * ((2 * hh) ^ vsw));
        const i32x4 hi = *(const i32x4*)(vb + 16 * ((2 * hh + 1) ^ vsw));
        const i32x8 vf = (i32x8){lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
        acc[dt] = mfma_f8(vf, pb, acc[dt]);
      }
    }

    if (more2) {
      if constexpr (NKV == 2)
        asm volatile("s_waitcnt vmcnt(5) lgkmcnt(0)\n\ts_barrier" ::: "memory");
      else
        asm volatile("s_waitcnt vmcnt(3) lgkmcnt(0)\n\ts_barrier" ::: "memory");
    } else
      asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
  };
  for (int j = 0; j < j_end; j += 3) {
    block(j, std::integral_constant<int, 0>{});
    if (j + 1 < j_end) block(j + 1, std::integral_constant<int, 1>{});
    if (j + 2 < j_end) block(j + 2, std::integral_constant<int, 2>{});
  }
  // acc is read below only inside the divergent `qrow < N` branch; keep the loop's MFMAs out
  // of it (an MFMA under a partial EXEC mask loses the inactive lanes' operand rows).
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt) keep_live(acc[dt]);
  mfma_result_fence();

  // ---------- epilogue: O = acc * S / (l * 448) (+ V's mean with smooth_v, one fma) ----------
  // The row and lane half are formed again from the lane id (v_mbcnt), so that their values from
  // the top of the kernel need not stay live across the loop.
  const int lane_e = (int)__builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u));
  const int l32e = lane_e & 31, hhe = lane_e >> 5;
  const int qrow_e = q0 + l32e;
  if (qrow_e < N) {
    if (LSE && hhe == 0)
      LSE[(int64_t)bh * N + qrow_e] = row_lse(mc, l_i, sm_scale, s_qmu[32 * w + l32e]);
    const float inv = (l_i > 0.0f) ? __fdiv_rn(Sb, l_i * P_SCALE) : 0.0f;
    T* op = O + b * o_sb + hd * o_sh + (int64_t)qrow_e * o_sr;
    const float* vmp = VMEAN ? VMEAN + (int64_t)kvp * D : nullptr;
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int d = 32 * dt + 8 * g + 4 * hhe;
        T ov[4];
        if (vmp) {
          const float4 vm = *(const float4*)(vmp + d);
          ov[0] = (T)__builtin_fmaf(acc[dt][4 * g + 0], inv, vm.x);
          ov[1] = (T)__builtin_fmaf(acc[dt][4 * g + 1], inv, vm.y);
          ov[2] = (T)__builtin_fmaf(acc[dt][4 * g + 2], inv, vm.z);
          ov[3] = (T)__builtin_fmaf(acc[dt][4 * g + 3], inv, vm.w);
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e) ov[e] = (T)(acc[dt][4 * g + e] * inv);
        }
        uint2 packed;
        __builtin_memcpy(&packed, ov, 8);
        *(uint2*)(op + d) = packed;
      }
  }
}

// ---------------------------------------------------------------------------------------------
// Parity entry: Q quantization exactly as the main loop does it, written out.
// 1-D grid of ceil(N/32) * BH blocks of 64 threads: block bh * ceil(N/32) + t, lane (q, h) of the
// wave handles row 32 t + q of plane bh.
// ---------------------------------------------------------------------------------------------
template <typename T, bool QK_INT8, int D>
__global__ __launch_bounds__(64) void quant_q_kernel(const T* __restrict__ Q, int64_t q_sb,
                                                     int64_t q_sh, int64_t q_sr, int H, int N,
                                                     float sm_scale, u8* __restrict__ Q8,
                                                     float* __restrict__ SQ, float* __restrict__ CQ) {
  const int nqb = (N + 31) / 32;
  const int bh = blockIdx.x / nqb, b = bh / H, hd = bh - b * H;
  const int lane = threadIdx.x, l32 = lane & 31, hh = lane >> 5;
  const int qrow = (blockIdx.x - bh * nqb) * 32 + l32;
  QFrag<D> qf;
  float sq, cq;
  quant_q_row<T, QK_INT8, D>(Q + b * q_sb + hd * q_sh + (int64_t)qrow * q_sr, qrow < N, hh,
                             sm_scale, qf, sq, cq);
  if (qrow >= N) return;
  u8* dst = Q8 + ((int64_t)bh * N + qrow) * D;
  if (QK_INT8) {
#pragma unroll
    for (int dd = 0; dd < D / 32; ++dd) *(i32x4*)(dst + 32 * dd + 16 * hh) = qf.i8[dd];
  } else {
#pragma unroll
    for (int dd = 0; dd < D / 64; ++dd) {
      const i32x8 v = qf.f8[dd];
      *(i32x4*)(dst + 64 * dd + 32 * hh) = (i32x4){v[0], v[1], v[2], v[3]};
      *(i32x4*)(dst + 64 * dd + 32 * hh + 16) = (i32x4){v[4], v[5], v[6], v[7]};
    }
  }
  if (hh == 0) {
    SQ[(int64_t)bh * N + qrow] = sq;
    CQ[(int64_t)bh * N + qrow] = cq;
  }
}

// ---------------------------------------------------------------------------------------------
// MFMA accumulator-layout probe: one wave, operands loaded in the main loop's fragment order
// (lane (r, h) holds row r, k-slots 16h.. (int8) or 32h.. (fp8)), results stored by the assumed
// 32x32 accumulator layout row = 8*(reg/4) + 4*(lane/32) + reg%4, column = lane%32.
// ---------------------------------------------------------------------------------------------
__global__ __launch_bounds__(64) void layout_probe_kernel(const u8* __restrict__ A,
                                                          const u8* __restrict__ BT,
                                                          int32_t* __restrict__ C,
                                                          const u8* __restrict__ E,
                                                          const u8* __restrict__ FT,
                                                          float* __restrict__ D) {
  const int lane = threadIdx.x, r = lane & 31, h = lane >> 5;
  const i32x4 a = *(const i32x4*)(A + r * 32 + 16 * h);
  const i32x4 bt = *(const i32x4*)(BT + r * 32 + 16 * h);
  i32x16 c;
#pragma unroll
  for (int i = 0; i < 16; ++i) c[i] = 0;
  c = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, bt, c, 0, 0, 0);
  const i32x8 e = *(const i32x8*)(E + r * 64 + 32 * h);
  const i32x8 ft = *(const i32x8*)(FT + r * 64 + 32 * h);
  f32x16 d;
#pragma unroll
  for (int i = 0; i < 16; ++i) d[i] = 0.0f;
  d = mfma_f8(e, ft, d);
  mfma_result_fence();   // the stores below read the results
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int row = 8 * (i >> 2) + 4 * h + (i & 3);
    C[row * 32 + r] = c[i];
    D[row * 32 + r] = d[i];
  }
}

// ---------------------------------------------------------------------------------------------
// MFMA throughput probe (benchmark only): the dense rate of the two matrix instructions the main
// loop issues, measured on this GPU at the clock it runs at. Every wave issues `iters` rounds of
// PEAK_NACC independent register-resident MFMAs (int8 32x32x32, or e4m3 32x32x64 with unit
// scales) on operands that are neither zero nor equal across lanes, so the matrix core's data
// paths toggle as on real data. Nothing is loaded: an asm statement that takes the accumulators
// in place (in AGPRs), after 64 wait states, keeps them live without any instruction reading
// them, and no wave ends with an MFMA in flight. With `clocks`, the first wave stores the
// shader-clock cycles (s_memtime) and constant-rate ticks (s_memrealtime) it spent.
// Ops per launch: blocks * 4 waves * iters * PEAK_NACC * 2*32*32*K (K = 32 int8, 64 e4m3).
// ---------------------------------------------------------------------------------------------
constexpr int PEAK_NACC = 4;

template <bool INT8>
__global__ __launch_bounds__(256) void mfma_peak_kernel(int64_t iters, int64_t* __restrict__ clocks) {
  const unsigned lane = threadIdx.x & 63;
  const uint64_t c0 = __builtin_amdgcn_s_memtime(), r0 = __builtin_amdgcn_s_memrealtime();
  if constexpr (INT8) {
    i32x4 a, b;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      a[i] = (int)(0x9E3779B9u * (4 * lane + i + 1));
      b[i] = (int)(0x85EBCA6Bu * (4 * lane + i + 7));
    }
    i32x16 acc[PEAK_NACC];
#pragma unroll
    for (int t = 0; t < PEAK_NACC; ++t)
#pragma unroll
      for (int i = 0; i < 16; ++i) acc[t][i] = 0;
    int64_t it = iters;   // >= 1 (the entry point checks)
    do {
#pragma unroll
      for (int t = 0; t < PEAK_NACC; ++t)
        acc[t] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, acc[t], 0, 0, 0);
    } while (--it > 0);
    // 64 wait states, then the results are taken in place by an empty statement (no read)
    asm volatile("s_nop 15\n s_nop 15\n s_nop 15\n s_nop 15"
                 : "+a"(acc[0]), "+a"(acc[1]), "+a"(acc[2]), "+a"(acc[3]));
  } else {
    // bytes masked with 0x57: e4m3 values with exponent field <= 10 -- finite, never NaN
    i32x8 a, b;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      a[i] = (int)((0x9E3779B9u * (8 * lane + i + 1)) & 0x57575757u);
      b[i] = (int)((0x85EBCA6Bu * (8 * lane + i + 7)) & 0x57575757u);
    }
    f32x16 acc[PEAK_NACC];
#pragma unroll
    for (int t = 0; t < PEAK_NACC; ++t)
#pragma unroll
      for (int i = 0; i < 16; ++i) acc[t][i] = 0.0f;
    int64_t it = iters;
    do {
#pragma unroll
      for (int t = 0; t < PEAK_NACC; ++t) acc[t] = mfma_f8(a, b, acc[t]);
    } while (--it > 0);
    asm volatile("s_nop 15\n s_nop 15\n s_nop 15\n s_nop 15"
                 : "+a"(acc[0]), "+a"(acc[1]), "+a"(acc[2]), "+a"(acc[3]));
  }
  // the shader-clock cycles and constant-rate ticks the first wave spent: the clock it ran at
  const uint64_t c1 = __builtin_amdgcn_s_memtime(), r1 = __builtin_amdgcn_s_memrealtime();
  if (clocks != nullptr && blockIdx.x == 0 && threadIdx.x == 0) {
    clocks[0] = (int64_t)(c1 - c0);
    clocks[1] = (int64_t)(r1 - r0);
  }
}

// ---------------------------------------------------------------------------------------------
template <typename T, bool QK_INT8, bool CAUSAL, int D>
static void launch_attn_d(const AttnArgs& a, hipStream_t stream) {
  const int BH = (int)(a.B * a.H);
  const int num_qt = (int)((a.N + BM - 1) / BM);
  const int total = num_qt * BH;
  const int span = (total / 8) * 8;
  hipLaunchKernelGGL((attn_fwd_kernel<T, QK_INT8, CAUSAL, D>), dim3(total), dim3(AT), 0, stream,
                     (const T*)a.q, (const u8*)a.k8, a.kconst, (const u8*)a.v8t, a.s, (T*)a.o,
                     a.q_sb, a.q_sh, a.q_sr, a.o_sb, a.o_sh, a.o_sr, (int)a.H, (int)a.H_kv,
                     (int)(a.H / a.H_kv), (int)a.N, (int)a.N_kv, (int)a.N_kv_pad, num_qt, span,
                     a.sm_scale, a.lse, a.kmean, a.vmean);
}

template <typename T, bool QK_INT8, bool CAUSAL>
static void launch_attn_t(const AttnArgs& a, hipStream_t stream) {
  if (a.D == 64) {
    launch_attn_d<T, QK_INT8, CAUSAL, 64>(a, stream);
  } else {
    launch_attn_d<T, QK_INT8, CAUSAL, 128>(a, stream);
  }
}

hipError_t launch_attn_fwd(const AttnArgs& a, hipStream_t stream) {
  if (a.dtype == 1) {
    if (a.causal)
      launch_attn_t<bf16, false, true>(a, stream);
    else
      launch_attn_t<bf16, false, false>(a, stream);
  } else if (a.qk_int8) {
    if (a.causal)
      launch_attn_t<f16, true, true>(a, stream);
    else
      launch_attn_t<f16, true, false>(a, stream);
  } else {
    if (a.causal)
      launch_attn_t<f16, false, true>(a, stream);
    else
      launch_attn_t<f16, false, false>(a, stream);
  }
  return hipGetLastError();
}

template <typename T, bool QK_INT8, int D>
static void launch_quant_q_t(const QuantQArgs& a, hipStream_t stream) {
  const dim3 grid((unsigned)((a.N + 31) / 32 * a.B * a.H));
  hipLaunchKernelGGL((quant_q_kernel<T, QK_INT8, D>), grid, dim3(64), 0, stream, (const T*)a.q,
                     a.q_sb, a.q_sh, a.q_sr, (int)a.H, (int)a.N, a.sm_scale, (u8*)a.q8, a.sq,
                     a.cq);
}

template <int D>
static void launch_quant_q_d(const QuantQArgs& a, hipStream_t stream) {
  if (a.dtype == 1)
    launch_quant_q_t<bf16, false, D>(a, stream);
  else if (a.qk_int8)
    launch_quant_q_t<f16, true, D>(a, stream);
  else
    launch_quant_q_t<f16, false, D>(a, stream);
}

hipError_t launch_quant_q(const QuantQArgs& a, hipStream_t stream) {
  if (a.D == 64)
    launch_quant_q_d<64>(a, stream);
  else
    launch_quant_q_d<128>(a, stream);
  return hipGetLastError();
}

hipError_t launch_layout_probe(const void* a, const void* bt, int32_t* c, const void* e,
                               const void* ft, float* d, hipStream_t stream) {
  hipLaunchKernelGGL(layout_probe_kernel, dim3(1), dim3(64), 0, stream, (const u8*)a,
                     (const u8*)bt, c, (const u8*)e, (const u8*)ft, d);
  return hipGetLastError();
}

hipError_t launch_mfma_peak(bool int8, int64_t blocks, int64_t iters, int64_t* clocks,
                            hipStream_t stream) {
  if (int8)
    hipLaunchKernelGGL(mfma_peak_kernel<true>, dim3((unsigned)blocks), dim3(256), 0, stream, iters,
                       clocks);
  else
    hipLaunchKernelGGL(mfma_peak_kernel<false>, dim3((unsigned)blocks), dim3(256), 0, stream, iters,
                       clocks);
  return hipGetLastError();
}

}  // namespace sage
