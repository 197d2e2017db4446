// The quantized flash-attention main loop on gfx950 (CDNA4, wave64 MFMA).
//
// Scheme (the reference's, kernels/hip/sk1_t6i.hip:84-299 and sk1_t4a1s.hip): Q is quantized per
// row inside the kernel (int8 for fp16 inputs, e4m3 for bf16), K8/SK/V8T/SV'/S come from the
// prologue. Per 64-key block: scores s = fp32(Q8.K8) * (c_q * SK), one running-max update, p =
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
// * K/V tiles are double-buffered in LDS with one barrier per block; the next block's global loads
//   are in flight during the current block's MFMAs. K rows use an XOR swizzle on 16-byte chunks,
//   V^T rows a 16-byte pad, so every MFMA operand read is bank-conflict free.
// * Causal: blocks past the CTA's diagonal are never visited, a wave skips blocks past its own
//   diagonal, and masks are applied only on diagonal blocks. The grid is a 1-D list of (plane,
//   q-tile) pairs, remapped so that each XCD (workgroup id mod 8) runs a contiguous range of
//   planes (K/V of a plane stay in that XCD's L2), longest causal tiles first.
#include "sage_device.h"
#include "sage_launch.h"

namespace sage {

constexpr int BM = 128;    // queries per block
constexpr int BK = 64;     // keys per main-loop step
constexpr int AT = 256;    // threads per block
constexpr int VROW = 80;   // LDS bytes per V^T row (64 keys + 16 pad)

// MFMA row r of score tile t (0/1) reads K row kappa(t, r) of the 64-key block. With the 32x32
// accumulator layout (row = 8*(reg/4) + 4*(lane/32) + reg%4), lane half h then holds keys
// 32h + 16t + reg.
__device__ __forceinline__ int kappa(int t, int r) {
  return 32 * ((r >> 2) & 1) + 16 * t + 4 * (r >> 3) + (r & 3);
}
// XOR swizzle of the 16-byte chunk position within a 128-byte K row.
__device__ __forceinline__ int kswz(int row) {
  return ((row >> 1) & 1) | ((((row)&1) ^ ((row >> 2) & 1)) << 1) | (((row >> 5) & 1) << 2);
}

// Q fragments of one query row, as the S^T MFMA's B operand wants them.
//   int8: 4 x 16 bytes, fragment dd = columns 32dd + 16h .. +15
//   fp8 : 2 x 32 bytes, fragment dd = columns 64dd + 32h .. +31
struct QFrag {
  i32x4 i8[4];
  i32x8 f8[2];
};

// Column of the c-th 8-element chunk a lane loads (c = 0..7), for lane half h.
template <bool QK_INT8>
__device__ __forceinline__ int qcol(int c, int h) {
  return QK_INT8 ? 32 * (c >> 1) + 16 * h + 8 * (c & 1) : 64 * (c >> 2) + 32 * h + 8 * (c & 3);
}

// Per-row Q quantization, shared by the main loop and the parity entry point.
// sk1_t6i.hip:91-117 (int8) and sk1_t4a1s.hip:79-105 (fp8):
//   amax = max(max_d |q|, 1e-12); qinv = RN(127/amax) (or 448); q8 = clamp(rne(RN(q*qinv)))
//   (fp8: e4m3(clamp(RN(q*qinv), +-448))); sq = RN(amax/127) (or 448); c_q = RN(RN(sm*log2e)*sq).
// Lanes q and q+32 hold the two halves of the row and exchange their partial absmax.
template <typename T, bool QK_INT8>
__device__ __forceinline__ void quant_q_row(const T* __restrict__ qrow_ptr, bool live, int h,
                                            float sm_scale, QFrag& qf, float& sq, float& cq) {
  float x[64];
#pragma unroll
  for (int c = 0; c < 8; ++c) {
    const u32x4 w = live ? *(const u32x4*)(qrow_ptr + qcol<QK_INT8>(c, h)) : (u32x4){0u, 0u, 0u, 0u};
    unpack8<T>(w, x + 8 * c);
  }
  float amax = 0.0f;
#pragma unroll
  for (int i = 0; i < 64; ++i) amax = fmaxf(amax, fabsf(x[i]));
  amax = fmaxf(amax, __shfl_xor(amax, 32, 64));
  amax = fmaxf(amax, SCALE_FLOOR);
  const float top = QK_INT8 ? I8_MAX : P_SCALE;
  const float qinv = __fdiv_rn(top, amax);
  sq = __fdiv_rn(amax, top);
  const float smlog = sm_scale * LOG2E_F;
  cq = smlog * sq;
  if (QK_INT8) {
#pragma unroll
    for (int dd = 0; dd < 4; ++dd) {
      const float* y = x + 16 * dd;
      qf.i8[dd] = (i32x4){(int)i8x4(y[0] * qinv, y[1] * qinv, y[2] * qinv, y[3] * qinv),
                          (int)i8x4(y[4] * qinv, y[5] * qinv, y[6] * qinv, y[7] * qinv),
                          (int)i8x4(y[8] * qinv, y[9] * qinv, y[10] * qinv, y[11] * qinv),
                          (int)i8x4(y[12] * qinv, y[13] * qinv, y[14] * qinv, y[15] * qinv)};
    }
  } else {
#pragma unroll
    for (int dd = 0; dd < 2; ++dd) {
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

__device__ __forceinline__ f32x16 mfma_f8(const i32x8 a, const i32x8 b, const f32x16 c) {
  // e4m3 x e4m3, unit e8m0 block scales (127 = 2^0).
  return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, c, 0, 0, 0, 127, 0, 127);
}

template <typename T, bool QK_INT8, bool CAUSAL>
__global__ __launch_bounds__(AT) __attribute__((amdgpu_waves_per_eu(2, 2))) void attn_fwd_kernel(
    const T* __restrict__ Q, const u8* __restrict__ K8, const float* __restrict__ SK,
    const u8* __restrict__ V8T, const float* __restrict__ SV, const float* __restrict__ Sfold,
    T* __restrict__ O, int64_t q_sb, int64_t q_sh, int64_t q_sr, int64_t o_sb, int64_t o_sh,
    int64_t o_sr, int H, int N, int N_pad, int num_qt, int xcd_span, float sm_scale) {
  __shared__ __attribute__((aligned(16))) u8 sK[2][BK * HD];
  __shared__ __attribute__((aligned(16))) u8 sV[2][HD * VROW];
  __shared__ __attribute__((aligned(16))) float sSK[2][BK];
  __shared__ __attribute__((aligned(16))) float sSV[2][BK];

  // ---- which (plane, q-tile) this block runs ----
  int id = blockIdx.x;
  if (id < xcd_span) id = (id & 7) * (xcd_span >> 3) + (id >> 3);
  const int bh = id / num_qt;
  int qt = id - bh * num_qt;
  if (CAUSAL) qt = num_qt - 1 - qt;
  const int b = bh / H, hd = bh - b * H;

  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int l32 = lane & 31, hh = lane >> 5;
  const int q0 = qt * BM + w * 32;
  const int qrow = q0 + l32;

  // ---- Q: per-row quantization straight into MFMA fragments ----
  QFrag qf;
  float sq, cq;
  quant_q_row<T, QK_INT8>(Q + b * q_sb + hd * q_sh + (int64_t)qrow * q_sr, qrow < N, hh, sm_scale,
                          qf, sq, cq);
  (void)sq;

  const u8* Kb = K8 + (int64_t)bh * N_pad * HD;
  const u8* Vb = V8T + (int64_t)bh * HD * N_pad;
  const float* SKb = SK + (int64_t)bh * N_pad;
  const float* SVb = SV + (int64_t)bh * N_pad;
  const float Sb = Sfold[bh];

  const int n_blocks = N_pad / BK;
  const int j_end = CAUSAL ? min(n_blocks, (qt * BM + BM - 1) / BK + 1) : n_blocks;
  const int w_end = CAUSAL ? min(j_end, (q0 + 31) / BK + 1) : j_end;

  // ---- staging: global -> registers -> LDS ----
  u32x4 kr0, kr1, vr0, vr1;
  f32x4 sr = {0.f, 0.f, 0.f, 0.f};
  auto gload = [&](int j) {
    const u8* kp = Kb + (int64_t)(BK * j + (tid >> 2)) * HD + 32 * (tid & 3);
    kr0 = *(const u32x4*)kp;
    kr1 = *(const u32x4*)(kp + 16);
    const u8* vp = Vb + (int64_t)(tid >> 1) * N_pad + BK * j + 32 * (tid & 1);
    vr0 = *(const u32x4*)vp;
    vr1 = *(const u32x4*)(vp + 16);
    if (tid < 16)
      sr = *(const f32x4*)(SKb + BK * j + 4 * tid);
    else if (tid < 32)
      sr = *(const f32x4*)(SVb + BK * j + 4 * (tid - 16)) * P_SCALE;
  };
  auto lstore = [&](int s) {
    const int row = tid >> 2, c0 = 2 * (tid & 3), sw = kswz(row);
    *(u32x4*)&sK[s][row * HD + 16 * (c0 ^ sw)] = kr0;
    *(u32x4*)&sK[s][row * HD + 16 * ((c0 + 1) ^ sw)] = kr1;
    u8* vd = &sV[s][(tid >> 1) * VROW + 32 * (tid & 1)];
    *(u32x4*)vd = vr0;
    *(u32x4*)(vd + 16) = vr1;
    if (tid < 16)
      *(f32x4*)&sSK[s][4 * tid] = sr;
    else if (tid < 32)
      *(f32x4*)&sSV[s][4 * (tid - 16)] = sr;
  };

  f32x16 acc[4];
#pragma unroll
  for (int dt = 0; dt < 4; ++dt)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[dt][r] = 0.0f;
  float m_i = -INFINITY, l_i = 0.0f;

  // MFMA row of this lane in the S^T tiles, and its swizzled K rows.
  const int krow0 = kappa(0, l32), krow1 = kappa(1, l32);
  const int ksw0 = kswz(krow0), ksw1 = kswz(krow1);

  gload(0);
  lstore(0);
  __syncthreads();

  for (int j = 0; j < j_end; ++j) {
    const int s = j & 1;
    const bool more = (j + 1 < j_end);
    if (more) gload(j + 1);

    if (!CAUSAL || j < w_end) {
      // ---------- S^T = K . Q^T for 64 keys: two 32x32 tiles ----------
      float sc[32];
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const int krow = t ? krow1 : krow0;
        const int ksw = t ? ksw1 : ksw0;
        const u8* kb = &sK[s][krow * HD];
        if (QK_INT8) {
          i32x16 a;
#pragma unroll
          for (int r = 0; r < 16; ++r) a[r] = 0;
#pragma unroll
          for (int dd = 0; dd < 4; ++dd) {
            const i32x4 kf = *(const i32x4*)(kb + 16 * ((2 * dd + hh) ^ ksw));
            a = __builtin_amdgcn_mfma_i32_32x32x32_i8(kf, qf.i8[dd], a, 0, 0, 0);
          }
#pragma unroll
          for (int r = 0; r < 16; ++r) sc[16 * t + r] = (float)a[r];
        } else {
          f32x16 a;
#pragma unroll
          for (int r = 0; r < 16; ++r) a[r] = 0.0f;
#pragma unroll
          for (int dd = 0; dd < 2; ++dd) {
            const int c0 = 4 * dd + 2 * hh;
            const i32x4 lo = *(const i32x4*)(kb + 16 * (c0 ^ ksw));
            const i32x4 hi = *(const i32x4*)(kb + 16 * ((c0 + 1) ^ ksw));
            const i32x8 kf = (i32x8){lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
            a = mfma_f8(kf, qf.f8[dd], a);
          }
#pragma unroll
          for (int r = 0; r < 16; ++r) sc[16 * t + r] = a[r];
        }
      }
      // ---------- scale, mask, one row max per 64 keys ----------
      const float* skb = &sSK[s][32 * hh];
#pragma unroll
      for (int k4 = 0; k4 < 8; ++k4) {
        const f32x4 kv = *(const f32x4*)(skb + 4 * k4);
#pragma unroll
        for (int e = 0; e < 4; ++e) sc[4 * k4 + e] = sc[4 * k4 + e] * (cq * kv[e]);
      }
      const bool need_mask = CAUSAL ? (BK * j + BK - 1 > q0) : (BK * j + BK > N);
      if (need_mask) {
        const int key0 = BK * j + 32 * hh;
#pragma unroll
        for (int i = 0; i < 32; ++i) {
          const int key = key0 + i;
          if (CAUSAL ? (key > qrow) : (key >= N)) sc[i] = -INFINITY;
        }
      }
      float lmax = sc[0];
#pragma unroll
      for (int i = 1; i < 32; ++i) lmax = fmaxf(lmax, sc[i]);
      lmax = fmaxf(lmax, __shfl_xor(lmax, 32, 64));
      const float m_new = fmaxf(m_i, lmax);
      const float m_use = (m_new == -INFINITY) ? 0.0f : m_new;
      const float alpha = __builtin_amdgcn_exp2f(m_i - m_use);
      m_i = m_new;

      // ---------- P = exp2(s - m), row sum, fold into e4m3 ----------
      const float* svb = &sSV[s][32 * hh];
      float psum = 0.0f;
      i32x8 pb;
#pragma unroll
      for (int k4 = 0; k4 < 8; ++k4) {
        const f32x4 vv = *(const f32x4*)(svb + 4 * k4);
        float p[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          p[e] = __builtin_amdgcn_exp2f(sc[4 * k4 + e] - m_use);
          psum += p[e];
          p[e] *= vv[e];
        }
        pb[k4] = (int)fp8x4(p[0], p[1], p[2], p[3]);
      }
      psum += __shfl_xor(psum, 32, 64);
      l_i = l_i * alpha + psum;
      if (__any(alpha != 1.0f)) {
#pragma unroll
        for (int dt = 0; dt < 4; ++dt)
#pragma unroll
          for (int r = 0; r < 16; ++r) acc[dt][r] *= alpha;
      }

      // ---------- O^T += V^T . P^T ----------
#pragma unroll
      for (int dt = 0; dt < 4; ++dt) {
        const u8* vb = &sV[s][(32 * dt + l32) * VROW + 32 * hh];
        const i32x4 lo = *(const i32x4*)vb;
        const i32x4 hi = *(const i32x4*)(vb + 16);
        const i32x8 vf = (i32x8){lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
        acc[dt] = mfma_f8(vf, pb, acc[dt]);
      }
    }

    if (more) lstore(s ^ 1);
    __syncthreads();
  }

  // ---------- epilogue: O = acc * S / (l * 448) ----------
  if (qrow < N) {
    const float inv = (l_i > 0.0f) ? __fdiv_rn(Sb, l_i * P_SCALE) : 0.0f;
    T* op = O + b * o_sb + hd * o_sh + (int64_t)qrow * o_sr;
#pragma unroll
    for (int dt = 0; dt < 4; ++dt)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int d = 32 * dt + 8 * g + 4 * hh;
        T ov[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) ov[e] = (T)(acc[dt][4 * g + e] * inv);
        uint2 packed;
        __builtin_memcpy(&packed, ov, 8);
        *(uint2*)(op + d) = packed;
      }
  }
}

// ---------------------------------------------------------------------------------------------
// Parity entry: Q quantization exactly as the main loop does it, written out.
// grid (ceil(N/32), BH), block 64: lane (q, h) of the wave handles row 32*blockIdx.x + q.
// ---------------------------------------------------------------------------------------------
template <typename T, bool QK_INT8>
__global__ __launch_bounds__(64) void quant_q_kernel(const T* __restrict__ Q, int64_t q_sb,
                                                     int64_t q_sh, int64_t q_sr, int H, int N,
                                                     float sm_scale, u8* __restrict__ Q8,
                                                     float* __restrict__ SQ, float* __restrict__ CQ) {
  const int bh = blockIdx.y, b = bh / H, hd = bh - b * H;
  const int lane = threadIdx.x, l32 = lane & 31, hh = lane >> 5;
  const int qrow = blockIdx.x * 32 + l32;
  QFrag qf;
  float sq, cq;
  quant_q_row<T, QK_INT8>(Q + b * q_sb + hd * q_sh + (int64_t)qrow * q_sr, qrow < N, hh, sm_scale,
                          qf, sq, cq);
  if (qrow >= N) return;
  u8* dst = Q8 + ((int64_t)bh * N + qrow) * HD;
  if (QK_INT8) {
#pragma unroll
    for (int dd = 0; dd < 4; ++dd) *(i32x4*)(dst + 32 * dd + 16 * hh) = qf.i8[dd];
  } else {
#pragma unroll
    for (int dd = 0; dd < 2; ++dd) {
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
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int row = 8 * (i >> 2) + 4 * h + (i & 3);
    C[row * 32 + r] = c[i];
    D[row * 32 + r] = d[i];
  }
}

// ---------------------------------------------------------------------------------------------
template <typename T, bool QK_INT8, bool CAUSAL>
static void launch_attn_t(const AttnArgs& a, hipStream_t stream) {
  const int BH = (int)(a.B * a.H);
  const int num_qt = (int)((a.N + BM - 1) / BM);
  const int total = num_qt * BH;
  const int span = (total / 8) * 8;
  hipLaunchKernelGGL((attn_fwd_kernel<T, QK_INT8, CAUSAL>), dim3(total), dim3(AT), 0, stream,
                     (const T*)a.q, (const u8*)a.k8, a.sk, (const u8*)a.v8t, a.sv, a.s, (T*)a.o,
                     a.q_sb, a.q_sh, a.q_sr, a.o_sb, a.o_sh, a.o_sr, (int)a.H, (int)a.N,
                     (int)a.N_pad, num_qt, span, a.sm_scale);
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

hipError_t launch_quant_q(const QuantQArgs& a, hipStream_t stream) {
  const dim3 grid((unsigned)((a.N + 31) / 32), (unsigned)(a.B * a.H));
  if (a.dtype == 1)
    hipLaunchKernelGGL((quant_q_kernel<bf16, false>), grid, dim3(64), 0, stream,
                       (const bf16*)a.q, a.q_sb, a.q_sh, a.q_sr, (int)a.H, (int)a.N, a.sm_scale,
                       (u8*)a.q8, a.sq, a.cq);
  else if (a.qk_int8)
    hipLaunchKernelGGL((quant_q_kernel<f16, true>), grid, dim3(64), 0, stream, (const f16*)a.q,
                       a.q_sb, a.q_sh, a.q_sr, (int)a.H, (int)a.N, a.sm_scale, (u8*)a.q8, a.sq,
                       a.cq);
  else
    hipLaunchKernelGGL((quant_q_kernel<f16, false>), grid, dim3(64), 0, stream, (const f16*)a.q,
                       a.q_sb, a.q_sh, a.q_sr, (int)a.H, (int)a.N, a.sm_scale, (u8*)a.q8, a.sq,
                       a.cq);
  return hipGetLastError();
}

hipError_t launch_layout_probe(const void* a, const void* bt, int32_t* c, const void* e,
                               const void* ft, float* d, hipStream_t stream) {
  hipLaunchKernelGGL(layout_probe_kernel, dim3(1), dim3(64), 0, stream, (const u8*)a,
                     (const u8*)bt, c, (const u8*)e, (const u8*)ft, d);
  return hipGetLastError();
}

}  // namespace sage
