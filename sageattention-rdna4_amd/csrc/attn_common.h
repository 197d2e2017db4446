// Device pieces shared by the 32-query-per-wave main loops (attn_fwd.hip, attn_fwd_pp.hip) and
// the Q parity entry: tile geometry, operand swizzles, the per-row Q quantizer, MFMA wrappers,
// the per-block online softmax.
#pragma once
#include <type_traits>

#include "sage_device.h"

namespace sage {

constexpr int BM = 128;    // queries per block
constexpr int BK = 64;     // keys per main-loop step
constexpr int AT = 256;    // threads per block
// Waves per SIMD the 128-query kernel's register budget is sized for: 3 for head_dim 128 (168
// VGPRs; three 52 KB blocks per CU), 4 for head_dim 64 (128 VGPRs; four 27 KB blocks). A third
// (fourth) wave fills the issue slots one wave's dependent softmax chain leaves empty: measured
// 3.7 % (6.4 %) faster than two waves, a few spilled registers at D = 128 included.
constexpr int attn_waves(int D) { return D == 64 ? 4 : 3; }


// MFMA row r of score tile t (0/1) reads K row kappa(t, r) of the 64-key block. With the 32x32
// accumulator layout (row = 8*(reg/4) + 4*(lane/32) + reg%4), lane half h then holds keys
// 32h + 16t + reg.
__device__ __forceinline__ int kappa(int t, int r) {
  return 32 * ((r >> 2) & 1) + 16 * t + 4 * (r >> 3) + (r & 3);
}
// XOR swizzle of the 16-byte chunk position within a K row of D bytes (8 chunks for D = 128, 4
// for D = 64). The 16 lanes of one LDS read pass hold rows {0..7, 32..39} + 16t (kappa), so the
// swizzle must separate rows that share a bank group: bits 2 and 5 of the row (and bit 1 / bit 0
// for the 128-byte row's 8 chunks).
template <int D = HD>
__device__ __forceinline__ int kswz(int row) {
  if (D == 64) return ((row >> 2) & 1) | (((row >> 5) & 1) << 1);
  return ((row >> 1) & 1) | ((((row)&1) ^ ((row >> 2) & 1)) << 1) | (((row >> 5) & 1) << 2);
}
// XOR swizzle of the 16-byte chunk position within a 64-byte V^T row: bits 2-3 of the row. A P.V
// operand read has lane l on row d = l % 32 + 32 dt, chunk 2 (l / 32) + half. Measured on gfx950
// (8 such ds_read_b128 per wave, 4 waves per CU): 219 cycles with this swizzle or bits 3-4, as for
// a linear read; 261 with ((d >> 1) ^ (d >> 3)) & 3, which maps rows d and d + 4 to the same two
// chunk slots, and 512 with none. So a read pass takes lanes from both halves of the wave.
__device__ __forceinline__ int vswz(int d) { return (d >> 2) & 3; }

// Q fragments of one query row of D columns, as the S^T MFMA's B operand wants them.
//   int8: D/32 x 16 bytes, fragment dd = columns 32dd + 16h .. +15
//   fp8 : D/64 x 32 bytes, fragment dd = columns 64dd + 32h .. +31
template <int D = HD>
struct QFrag {
  i32x4 i8[D / 32];
  i32x8 f8[D / 64];
};

// Column of the c-th 8-element chunk a lane loads (c = 0 .. D/16 - 1), for lane half h.
template <bool QK_INT8>
__device__ __forceinline__ int qcol(int c, int h) {
  return QK_INT8 ? 32 * (c >> 1) + 16 * h + 8 * (c & 1) : 64 * (c >> 2) + 32 * h + 8 * (c & 3);
}

// Per-row Q quantization, shared by the main loop and the parity entry point.
// sk1_t6i.hip:91-117 (int8) and sk1_t4a1s.hip:79-105 (fp8):
//   amax = max(max_d |q|, 1e-12); qinv = RN(127/amax) (or 448); q8 = clamp(rne(RN(q*qinv)))
//   (fp8: e4m3(clamp(RN(q*qinv), +-448))); sq = RN(amax/127) (or 448); c_q = RN(RN(sm*log2e)*sq).
// Lanes q and q+32 hold the two halves of the row and exchange their partial absmax.
// With `mu` (the plane's smooth_k mean, 128 fp32), also returns q . mu over the whole row in
// `qmu` (fp32 products and sums, both lanes get it): the row's logsumexp correction for smooth_k.
template <typename T, bool QK_INT8, int D = HD>
__device__ __forceinline__ void quant_q_row(const T* __restrict__ qrow_ptr, bool live, int h,
                                            float sm_scale, QFrag<D>& qf, float& sq, float& cq,
                                            const float* __restrict__ mu = nullptr,
                                            float* qmu = nullptr) {
  constexpr int NC = D / 16;   // 8-element chunks per lane (half a row)
  float x[D / 2];
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    const u32x4 w = live ? *(const u32x4*)(qrow_ptr + qcol<QK_INT8>(c, h)) : (u32x4){0u, 0u, 0u, 0u};
    unpack8<T>(w, x + 8 * c);
  }
  if (mu) {
    float d = 0.0f;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const f32x4 m0 = *(const f32x4*)(mu + qcol<QK_INT8>(c, h));
      const f32x4 m1 = *(const f32x4*)(mu + qcol<QK_INT8>(c, h) + 4);
#pragma unroll
      for (int e = 0; e < 4; ++e) d = __builtin_fmaf(x[8 * c + e], m0[e], d);
#pragma unroll
      for (int e = 0; e < 4; ++e) d = __builtin_fmaf(x[8 * c + 4 + e], m1[e], d);
    }
    *qmu = d + __shfl_xor(d, 32, 64);
  }
  float amax = 0.0f;
#pragma unroll
  for (int i = 0; i < D / 2; ++i) amax = fmaxf(amax, fabsf(x[i]));
  amax = fmaxf(amax, __shfl_xor(amax, 32, 64));
  amax = fmaxf(amax, SCALE_FLOOR);
  const float top = QK_INT8 ? I8_MAX : P_SCALE;
  const float qinv = __fdiv_rn(top, amax);
  sq = __fdiv_rn(amax, top);
  const float smlog = sm_scale * LOG2E_F;
  cq = smlog * sq;
  if (QK_INT8) {
#pragma unroll
    for (int dd = 0; dd < D / 32; ++dd) {
      const float* y = x + 16 * dd;
      qf.i8[dd] = (i32x4){(int)i8x4(y[0] * qinv, y[1] * qinv, y[2] * qinv, y[3] * qinv),
                          (int)i8x4(y[4] * qinv, y[5] * qinv, y[6] * qinv, y[7] * qinv),
                          (int)i8x4(y[8] * qinv, y[9] * qinv, y[10] * qinv, y[11] * qinv),
                          (int)i8x4(y[12] * qinv, y[13] * qinv, y[14] * qinv, y[15] * qinv)};
    }
  } else {
#pragma unroll
    for (int dd = 0; dd < D / 64; ++dd) {
      const float* y = x + 32 * dd;
      float z[32];
#pragma unroll
      for (int i = 0; i < 32; ++i) z[i] = fminf(fmaxf(y[i] * qinv, -P_SCALE), P_SCALE);
#pragma unroll
      for (int k = 0; k < 8; ++k)
        qf.f8[dd][k] = (int)fp8x4(z[4 * k], z[4 * k + 1], z[4 * k + 2], z[4 * k + 3]);
    }
  }
}

typedef __attribute__((address_space(3))) void lds_void_t;
typedef __attribute__((address_space(1))) void glb_void_t;

// 16 bytes per lane, global -> LDS, bypassing registers: lane i of the wave lands at
// lds_wave_base + 16 * i (the LDS base must be the same for the whole wave).
__device__ __forceinline__ void g2lds16(const void* src, void* lds_wave_base) {
  __builtin_amdgcn_global_load_lds((glb_void_t*)src, (lds_void_t*)lds_wave_base, 16, 0, 0);
}

// LDS byte address of a pointer into __shared__ memory.
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(const lds_void_t*)p;
}

// The same moves written as instructions the compiler does not see, for a loop that keeps its own
// count of them: global address = uniform 64-bit base + per-lane 32-bit offset, LDS destination
// = uniform lds base + 16 * lane (dwordx4) or + 4 * lane (dword). The compiler then neither waits
// for them (the caller's s_waitcnt does, before the barrier that publishes the data) nor spends
// per-lane 64-bit adds on the addresses. Any of its own vector-memory waits stay correct: the
// counter retires in order, so extra operations in flight only make its waits longer.
__device__ __forceinline__ void dma16(const void* base, uint32_t voff, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1"
               :: "v"(voff), "s"(base), "s"(lds) : "memory", "m0");
}
__device__ __forceinline__ void dma4(const void* base, uint32_t voff, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dword %0, %1"
               :: "v"(voff), "s"(base), "s"(lds) : "memory", "m0");
}

// Keeps an accumulator tile live (in registers, computed) at this point. A separate function with
// a fixed operand type: the same empty asm written on an array element of template-dependent size
// fails the host pass's constraint check, and that failure is silent there -- the kernel's host
// stub is dropped and the library has an undefined symbol.
__device__ __forceinline__ void keep_live(const f32x16& v) { asm volatile("" ::"v"(v)); }

__device__ __forceinline__ f32x16 mfma_f8(const i32x8 a, const i32x8 b, const f32x16 c) {
  // e4m3 x e4m3, unit e8m0 block scales (127 = 2^0).
  return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, c, 0, 0, 0, 127, 0, 127);
}

// Score tile pair of one 64-key block: st[t][reg] holds, for lane (q, h), the raw MFMA result for
// key 32h + 16t + reg -- int8: the bits of the int32 Q8.K8; fp8: the fp32 dot product.
template <bool QK_INT8, int D = HD>
__device__ __forceinline__ void qk_block(const u8* __restrict__ kbuf, const QFrag<D>& qf,
                                         int krow0, int krow1, int ksw0, int ksw1, int hh,
                                         f32x16 (&st)[2]) {
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    const int krow = t ? krow1 : krow0;
    const int ksw = t ? ksw1 : ksw0;
    const u8* kb = kbuf + krow * D;
    if (QK_INT8) {
      i32x16 a;
#pragma unroll
      for (int r = 0; r < 16; ++r) a[r] = 0;
#pragma unroll
      for (int dd = 0; dd < D / 32; ++dd) {
        const i32x4 kf = *(const i32x4*)(kb + 16 * ((2 * dd + hh) ^ ksw));
        a = __builtin_amdgcn_mfma_i32_32x32x32_i8(kf, qf.i8[dd], a, 0, 0, 0);
      }
      st[t] = __builtin_bit_cast(f32x16, a);
    } else {
      f32x16 a;
#pragma unroll
      for (int r = 0; r < 16; ++r) a[r] = 0.0f;
#pragma unroll
      for (int dd = 0; dd < D / 64; ++dd) {
        const int c0 = 4 * dd + 2 * hh;
        const i32x4 lo = *(const i32x4*)(kb + 16 * (c0 ^ ksw));
        const i32x4 hi = *(const i32x4*)(kb + 16 * ((c0 + 1) ^ ksw));
        const i32x8 kf = (i32x8){lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
        a = mfma_f8(kf, qf.f8[dd], a);
      }
      st[t] = a;
    }
  }
}

// Per-key constants of one 64-key block in LDS, in the layout the prologue writes them (two rows
// of 64 fp32, 512 bytes per block): SK, then W = RN(SV' * 448).
struct ScaleTile {
  float sk[BK];
  float w[BK];
  float pad[2 * BK];   // landing area of the 128-query kernel's waves 2 and 3, whose copies keep
                       // every wave's request count equal
};

// Max of 32 values as 16 three-input maxima (v_max3_f32), a tree of depth 4.
__device__ __forceinline__ float max32(const float* x) {
  float m[10];
#pragma unroll
  for (int i = 0; i < 10; ++i) m[i] = fmaxf(fmaxf(x[3 * i], x[3 * i + 1]), x[3 * i + 2]);
  const float n0 = fmaxf(fmaxf(m[0], m[1]), m[2]);
  const float n1 = fmaxf(fmaxf(m[3], m[4]), m[5]);
  const float n2 = fmaxf(fmaxf(m[6], m[7]), m[8]);
  const float n3 = fmaxf(fmaxf(m[9], x[30]), x[31]);
  return fmaxf(fmaxf(fmaxf(n0, n1), n2), n3);
}

// One staging buffer of the main loop: a 64-key block's K tile (64 rows x D bytes, XOR-swizzled
// 16-byte chunks), V^T tile (D rows x 64 B, swizzled) and per-key constants.
template <int D = HD>
struct __attribute__((aligned(16))) StageBuf {
  u8 k[BK * D];
  u8 v[D * BK];
  ScaleTile s;
};

// Both 32-lane halves of a wave exchange values: returns (lower-half value, upper-half value) in
// every lane, with one v_permlane32_swap (no LDS round trip).
__device__ __forceinline__ float max_halves(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float sum_halves(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}


// Calls f(integral_constant<int, i>) for i = I .. N-1, unrolled (compile-time lane selectors).
template <int I, int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (I < N) {
    f(std::integral_constant<int, I>{});
    static_for<I + 1, N>(f);
  }
}

// Every lane receives lane n of its own 16-lane row (DPP row_newbcast:n). The compiler folds the
// move into the consuming VALU instruction (v_mul_f32_dpp ... row_newbcast:n).
template <int N>
__device__ __forceinline__ float row_bcast(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x150 + N, 0xF, 0xF, false));
}

// Per-key constants of one 64-key block, held as broadcast sources: lane l of half h = l/32
// holds SK and W of keys 32h + (l & 15) (sk0, w0) and 32h + 16 + (l & 15) (sk1, w1). Both 16-lane
// rows of a half hold the same values, so score jj of a lane (key 32h + jj) finds its constant in
// lane jj & 15 of its own row. Four 4-byte LDS reads per block instead of 32 floats per constant
// per lane.
struct KeyConsts {
  float sk0, sk1, w0, w1;
};
__device__ __forceinline__ KeyConsts load_key_consts(const ScaleTile& sc, int lane) {
  const int c = 32 * (lane >> 5) + (lane & 15);
  return {sc.sk[c], sc.sk[c + 16], sc.w[c], sc.w[c + 16]};
}

// The online softmax of one 64-key block for this lane's query (sk1_t6i.hip:162-279), in two
// halves that a pipelined loop can run for different blocks side by side.
//
// scores_block: x = fp32(Q8.K8) * SK, written over the raw scores (int8: the int32 dot products;
// fp8: already fp32); masked keys (causal: key > qrow; non-causal: key >= N) -inf; the running max
// m_new = max(m, max x); returns the block's shift mc = RN(c_q * m_new) (0 while m_new is -inf)
// and alpha = exp2(mc_prev - mc), exactly 1 when the max did not move (the reference's
// exp2(m - m)). A chain of dependent steps: the latency-bound half. q0: the wave's first query.
struct BlockShift {
  float mc, alpha;
};

// block_max: the first part of scores_block -- x = fp32(Q8.K8) * SK over the raw scores, masked
// keys -inf -- returning this lane's query's max over the block's 64 keys.
template <bool QK_INT8, bool CAUSAL, int NCONV = 0>
__device__ __forceinline__ float block_max(f32x16 (&sx)[2], float sk0, float sk1, int j, int q0,
                                           int qrow, int N, int hh) {
  static_for<0, 32>([&](auto ic) {
    constexpr int jj = decltype(ic)::value;
    const float v = sx[jj >> 4][jj & 15];
    const float d = (QK_INT8 && jj >= NCONV) ? (float)__float_as_int(v) : v;
    sx[jj >> 4][jj & 15] = d * row_bcast<jj & 15>(jj < 16 ? sk0 : sk1);
  });
  const bool need_mask = CAUSAL ? (BK * j + BK - 1 > q0) : (BK * j + BK > N);
  if (need_mask) {
    // key = key0 + i is dead when key > qrow (causal) or key >= N (tail): compare the constant
    // i against one per-lane limit.
    const int lim = (CAUSAL ? qrow + 1 : N) - (BK * j + 32 * hh);
#pragma unroll
    for (int i = 0; i < 32; ++i)
      if (i >= lim) sx[i >> 4][i & 15] = -INFINITY;
  }
  // max over the lane's 32 scores (16 three-input maxima), then across the two lane halves
  float x[32];
#pragma unroll
  for (int i = 0; i < 32; ++i) x[i] = sx[i >> 4][i & 15];
  return max_halves(max32(x));
}

// The exp2 shift of the running max m: c_q * m (0 while m is -inf), lowered by one to two ulps.
// With that, the max key's exp2 argument c_q*m - mc (exact in the fma) is never negative, and the
// probabilities' exp2 is clamped to at most 1, so the max key gets p = 1 exactly, as the
// reference's exp2(s - m) does. (With the shift RN(c_q*m) the argument is the product's rounding
// residual, +-1e-6, and p*W can then round to the other side of an e4m3 tie: a 6-8% change of the
// dominant key's weight.) 0 stays 0.
__device__ __forceinline__ float shift_of(float m, float cq) {
  float mc = cq * ((m == -INFINITY) ? 0.0f : m);
  mc = __builtin_fmaf(__builtin_fabsf(mc), -0x1p-23f, mc);
  // mc is rounded before it is used: the opaque copy keeps the compiler from fusing the products
  // into the subtraction that forms alpha, which it would do or not depending on the surrounding
  // code (so two kernels would round alpha differently). exp2(mc - mc_new) of the rounded shifts
  // is then exactly 1 for an unmoved max; the select skips the exp2 there.
  asm volatile("" : "+v"(mc));
  return mc;
}

template <bool QK_INT8, bool CAUSAL, int NCONV = 0>
__device__ __forceinline__ BlockShift scores_block(f32x16 (&sx)[2], float sk0, float sk1, int j, int q0,
                                                   int qrow, int N, int hh, float cq, float& m_x,
                                                   float& mc) {
  const float mx = block_max<QK_INT8, CAUSAL, NCONV>(sx, sk0, sk1, j, q0, qrow, N, hh);
  const float m_new = fmaxf(m_x, mx);
  const float mc_new = shift_of(m_new, cq);
  const float alpha = (m_new != m_x) ? __builtin_amdgcn_exp2f(mc - mc_new) : 1.0f;
  m_x = m_new;
  mc = mc_new;
  return {mc_new, alpha};
}

// int8 Q.K: the first NCONV of this lane's 32 raw int32 scores converted to fp32 in place (exact:
// |Q8.K8| <= 2^21), so that a scores_block<..., NCONV> that follows skips their conversion. Lets a
// kernel move the conversion out of the softmax's issue-bound stretch.
template <int NCONV>
__device__ __forceinline__ void convert_scores(f32x16 (&sx)[2]) {
  static_for<0, NCONV>([&](auto ic) {
    constexpr int jj = decltype(ic)::value;
    sx[jj >> 4][jj & 15] = (float)__float_as_int(sx[jj >> 4][jj & 15]);
  });
}

// O *= alpha before the block's P.V, skipped when every lane of the wave has alpha == 1.
template <int NDT>
__device__ __forceinline__ void rescale_acc(f32x16 (&acc)[NDT], float alpha) {
  if (__any(alpha != 1.0f)) {
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[dt][r] *= alpha;
  }
}

// 64 wait states before VALU code reads accumulators that P.V MFMAs may have just written (the
// epilogue). The compiler's own padding after v_mfma_scale_f32_32x32x64_f8f6f4 is 18 wait states,
// short of what the hardware takes to write the last pass of the result: in a main-loop variant
// whose last P.V was followed by register copies, a copy of registers 14-15 of the final tile made
// 18 wait states after the MFMA read stale values, nondeterministically (output channels 122,
// 123, 126 and 127).
__device__ __forceinline__ void mfma_result_fence() {
  __builtin_amdgcn_sched_barrier(0);
  asm volatile("s_nop 15\n\ts_nop 15\n\ts_nop 15\n\ts_nop 15" ::: "memory");
  __builtin_amdgcn_sched_barrier(0);
}
// The same for the duration of the 32x32x32 int8 MFMA (32 wait states), or of the MFMA that
// computed S^T: int8 Q.K (32) or e4m3 Q.K (64).
__device__ __forceinline__ void mfma_result_fence32() {
  __builtin_amdgcn_sched_barrier(0);
  asm volatile("s_nop 15\n\ts_nop 15" ::: "memory");
  __builtin_amdgcn_sched_barrier(0);
}
template <bool QK_INT8>
__device__ __forceinline__ void qk_result_fence() {
  if (QK_INT8)
    mfma_result_fence32();
  else
    mfma_result_fence();
}

// probs_block: p = exp2(c_q*x - mc); l = l*alpha + sum p (the row sum is taken before the fold);
// P8 = e4m3(p * RN(SV'*448)) into pb; with RESCALE, acc *= alpha (else the caller does it before
// the block's P.V). Independent steps: the throughput-bound half. w0/w1: the W broadcast sources.
template <bool RESCALE = true, int NDT = 4>
__device__ __forceinline__ void probs_block(const f32x16 (&x)[2], float w0, float w1, float cq,
                                            BlockShift sh, float& l_i, f32x16 (&acc)[NDT],
                                            i32x8& pb) {
  // W enters through an opaque copy: otherwise its broadcasts are hoisted above the preceding
  // branch, away from the multiplies they would fold into (one extra move per score).
  asm volatile("" : "+v"(w0), "+v"(w1));
  float ps[4];
  static_for<0, 8>([&](auto k4c) {
    constexpr int k4 = decltype(k4c)::value;
    float p[4];
    static_for<0, 4>([&](auto ec) {
      constexpr int e = decltype(ec)::value;
      constexpr int jj = 4 * k4 + e;
      // min(exp2, 1) through the VOP3 clamp bit of v_exp_f32 (no extra instruction)
      p[e] = __builtin_amdgcn_fmed3f(
          __builtin_amdgcn_exp2f(__builtin_fmaf(x[jj >> 4][jj & 15], cq, -sh.mc)), 0.0f, 1.0f);
      ps[e] = k4 ? ps[e] + p[e] : p[e];
      p[e] *= row_bcast<jj & 15>(jj < 16 ? w0 : w1);
    });
    pb[k4] = (int)fp8x4(p[0], p[1], p[2], p[3]);
  });
  // P is complete before the rescale branch (else its products sink past it, apart from the
  // broadcasts they would fold into)
  asm volatile("" ::"v"(pb));
  const float psum = sum_halves((ps[0] + ps[1]) + (ps[2] + ps[3]));
  l_i = __builtin_fmaf(l_i, sh.alpha, psum);
  if (RESCALE) rescale_acc(acc, sh.alpha);
}

// Both halves for one block, in order.
template <bool QK_INT8, bool CAUSAL, int NDT>
__device__ __forceinline__ void softmax_block(f32x16 (&st)[2], const KeyConsts& kc, int j, int q0,
                                              int qrow, int N, int hh, float cq, float& m_x,
                                              float& mc, float& l_i, f32x16 (&acc)[NDT],
                                              i32x8& pb) {
  const BlockShift sh =
      scores_block<QK_INT8, CAUSAL>(st, kc.sk0, kc.sk1, j, q0, qrow, N, hh, cq, m_x, mc);
  probs_block(st, kc.w0, kc.w1, cq, sh, l_i, acc, pb);
}


// S^T tile t of a 64-key block (keys 32h + 16t + reg of lane half h) for this lane's query:
// int8 -- the bits of the int32 Q8.K8; fp8 -- the fp32 dot product.
template <bool QK_INT8, int D>
__device__ __forceinline__ f32x16 qk_tile(const u8* __restrict__ kbuf, const QFrag<D>& qf, int krow,
                                          int ksw, int hh) {
  const u8* kb = kbuf + krow * D;
  if constexpr (QK_INT8) {
    i32x16 a;
#pragma unroll
    for (int r = 0; r < 16; ++r) a[r] = 0;
#pragma unroll
    for (int dd = 0; dd < D / 32; ++dd) {
      const i32x4 kf = *(const i32x4*)(kb + 16 * ((2 * dd + hh) ^ ksw));
      a = __builtin_amdgcn_mfma_i32_32x32x32_i8(kf, qf.i8[dd], a, 0, 0, 0);
    }
    return __builtin_bit_cast(f32x16, a);
  } else {
    f32x16 a;
#pragma unroll
    for (int r = 0; r < 16; ++r) a[r] = 0.0f;
#pragma unroll
    for (int dd = 0; dd < D / 64; ++dd) {
      const int c0 = 4 * dd + 2 * hh;
      const i32x4 lo = *(const i32x4*)(kb + 16 * (c0 ^ ksw));
      const i32x4 hi = *(const i32x4*)(kb + 16 * ((c0 + 1) ^ ksw));
      const i32x8 kf = (i32x8){lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
      a = mfma_f8(kf, qf.f8[dd], a);
    }
    return a;
  }
}

// The exponentials, row-sum partials and e4m3 P of the 16 scores of tile T (keys 32h + 16T + r):
// the same operations, in the same order per score and per partial sum, as probs_block
// (attn_common.h), which does both tiles in one pass. w: the tile's W broadcast source.
template <int T>
__device__ __forceinline__ void probs_tile(const f32x16 (&x)[2], float w, float cq, float mc,
                                           float (&ps)[4], i32x8& pb) {
  // W enters through an opaque copy: otherwise its broadcasts can be hoisted away from the
  // multiplies they fold into (one extra move, and a live register, per score)
  asm volatile("" : "+v"(w));
  static_for<0, 4>([&](auto k4c) {
    constexpr int k4 = decltype(k4c)::value + 4 * T;
    float p[4];
    static_for<0, 4>([&](auto ec) {
      constexpr int e = decltype(ec)::value;
      constexpr int jj = 4 * k4 + e;
      p[e] = __builtin_amdgcn_fmed3f(__builtin_amdgcn_exp2f(__builtin_fmaf(x[T][jj & 15], cq, -mc)),
                                     0.0f, 1.0f);
      ps[e] = k4 ? ps[e] + p[e] : p[e];
      p[e] *= row_bcast<jj & 15>(w);
    });
    pb[k4] = (int)fp8x4(p[0], p[1], p[2], p[3]);
  });
}

// The row's natural-log logsumexp of its scores times sm_scale, as the reference returns it
// (core.py:1437-1439): log2-domain sum RN(c_q*m) + log2(l), divided by 1.44269504, plus
// sm_scale * (q . mu) when the keys were smoothed.
__device__ __forceinline__ float row_lse(float mc, float l_i, float sm_scale, float qmu) {
  const float lse2 = mc + __builtin_amdgcn_logf(l_i);
  return __builtin_fmaf(sm_scale, qmu, __fdiv_rn(lse2, 1.44269504f));
}

}  // namespace sage
