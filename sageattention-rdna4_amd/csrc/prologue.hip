// The K/V prologue on gfx950: two launches, both HBM-bound streaming passes.
//
//   1. stats pass  (kv_stats_kernel):  reads K and V once (with smooth_v: twice, see VMode).
//        * K: per-column fp64 partial sums over the block's rows (the smooth_k mean), written to the
//          workspace as C1 partials per plane -- no atomics, so the sum order is fixed;
//        * V: per-token scale sv = max(RN(vmax/448), 1e-12), e4m3 quantization, and the transposed
//          store V8T[d][n] through an LDS tile; SV is written; the block's max sv goes to the
//          workspace for the fold.
//   2. quant pass  (k_quant_kernel):   reads K again.
//        * reduces the C1 mean partials of its plane in a fixed order (every block gets the same
//          bits), mu = fp32(sum / N);
//        * S = max(1, max sv) from the stats partials; SV' = RN(SV / S) in place for its rows;
//        * K per-token quantization: int8 (round half to even, clamp) or e4m3.
//
// The arithmetic restates kernels/hip/h34_prologue.hip:116-211 (K and V quantizers),
// :259-282 (fp64 mean) and sageattention/sk1_backend/__init__.py:561-579 (the S fold) of the
// reference. The mean is fp64-accumulated from exactly widened inputs like the reference's; the
// summation order differs, which cannot change the bits whenever the fp64 sum is exact (fp16 data
// of magnitude below 2^10 at N below 2^19 -- every served shape of interest).
//
// Thread layout of both passes: 256 threads = 16 column groups (cg, 8 columns = one 16-byte load)
// x 16 row groups (rg). The 16 lanes sharing a row are one aligned 16-lane group of a wave, so a
// row's absmax is four DPP max steps within the group (maxg).
#include "sage_device.h"
#include "sage_launch.h"

namespace sage {

constexpr int PT = 256;          // threads per block

// Thread layout of both passes for head_dim D: CG = D/8 column groups of 8 columns (one 16-byte
// load) x RG = 256/CG row groups; a row's CG lanes are one aligned CG-lane group of a wave. The
// stats pass moves STEP = 8*RG rows per step (8 consecutive tokens per thread: one 8-byte word of
// the transposed tile per column), through an LDS tile of D rows x (STEP + 16) bytes.
template <int D>
struct Geo {
  static constexpr int CG = D / 8, RG = PT / CG, STEP = 8 * RG, VTS = STEP + 16;
};

// Both grids are sized to one round of resident blocks on the device's compute units (a block is 4
// waves, one per SIMD; MI355X has 256 CUs): the stats pass fits 3 blocks per CU (at most 168
// VGPRs; its 16 row loads of 16 bytes per lane keep ~190 KB in flight per CU), the quant pass 8
// (at most 64 VGPRs). A partly filled second round costs a streaming pass as much as a full one.
// Each plane gets c = slots / BH blocks (at least 1) of equal row counts; a stats block's rows are
// a whole number of its steps (128 rows for head_dim 128, 256 for 64), so no step reaches into
// the next block's rows. A larger step, or fewer CUs, only lowers C1, so the head_dim-128
// geometry on MAX_CUS bounds the workspace for every call; a device with more CUs than that runs
// the MAX_CUS grids.
constexpr int64_t MAX_CUS = 256;
constexpr int64_t STATS_BLOCKS_PER_CU = 3;
constexpr int64_t QUANT_BLOCKS_PER_CU = 8;

PrologueGeom prologue_geom(int64_t BH, int64_t N, int64_t N_pad, int64_t step, int64_t cus) {
  auto cdiv = [](int64_t a, int64_t b) { return (a + b - 1) / b; };
  auto blocks_per_plane = [&](int64_t slots) { return BH < slots ? slots / BH : (int64_t)1; };
  const int64_t cu = (cus <= 0 || cus > MAX_CUS) ? MAX_CUS : cus;
  const int64_t Nc = cdiv(N, 64) * 64;
  PrologueGeom g;
  g.R1 = cdiv(cdiv(Nc, blocks_per_plane(cu * STATS_BLOCKS_PER_CU)), step) * step;
  g.C1 = cdiv(Nc, g.R1);
  g.R2 = cdiv(cdiv(N_pad, blocks_per_plane(cu * QUANT_BLOCKS_PER_CU)), 64) * 64;
  g.C2 = cdiv(N_pad, g.R2);
  return g;
}

// Workspace: K's mean partials, V's mean partials (smooth_v), the per-block max of sv -- each
// region 256-byte aligned. The V region is always reserved, so the size does not depend on flags.
static size_t part_region_bytes(int64_t BH, const PrologueGeom& g) {
  return ((size_t)BH * g.C1 * HD * sizeof(double) + 255) / 256 * 256;
}

size_t prologue_workspace_bytes(int64_t BH, int64_t N) {
  const int64_t Nc = (N + 63) / 64 * 64;
  const PrologueGeom g = prologue_geom(BH, N, Nc);
  const size_t smax = (size_t)BH * g.C1 * sizeof(float);
  return 2 * part_region_bytes(BH, g) + ((smax + 255) / 256 * 256);
}

// ---------------------------------------------------------------------------------------------
// Stats pass. grid (C1, BH), block 256.
// In a STEP-row step, thread (cg, rg) owns rows 8rg .. 8rg+7 and columns 8cg .. 8cg+7, so for each
// of its 8 columns it holds 8 consecutive tokens: one 8-byte word of the transposed tile. The LDS
// tile is [D d][STEP+16 B]; the 8-byte chunk of tokens 8rg..8rg+7 of row d sits at chunk position
// rg ^ (d >> 3), which keeps both the column writes and the row reads free of bank conflicts.
// ---------------------------------------------------------------------------------------------
// V_QUANT: V quantized as it is (and K's mean partials when smooth_k) -- the whole stats pass.
// V_SUMS: K's and V's mean partials only (smooth_v, first launch).
// V_CENTERED: V's mean from its partials (written to VMEAN), V - mean quantized (smooth_v, second
//             launch; K is not read).
// K_ONLY: K's mean partials only (the smooth_k mean on its own; V is not read).
enum VMode { V_QUANT = 0, V_SUMS = 1, V_CENTERED = 2, K_ONLY = 3 };

template <typename T, int VMODE, int D>
__global__ __launch_bounds__(PT) __attribute__((amdgpu_waves_per_eu(STATS_BLOCKS_PER_CU))) void kv_stats_kernel(
    const T* __restrict__ K, const T* __restrict__ V, u8* __restrict__ V8T, float* __restrict__ SV,
    double* __restrict__ part, double* __restrict__ vpart, float* __restrict__ VMEAN,
    float* __restrict__ smax, int64_t H, int64_t N, int64_t N_pad, int64_t R1, int64_t C1,
    int64_t k_sb, int64_t k_sh, int64_t k_sr, int64_t v_sb, int64_t v_sh, int64_t v_sr,
    int smooth_k) {
  using G = Geo<D>;
  constexpr int STEP = G::STEP, VT_STRIDE = G::VTS, RG = G::RG;
  __shared__ __attribute__((aligned(16))) u8 tile[D * VT_STRIDE];
  __shared__ float wmax[PT / 64];
  __shared__ float vmu_s[D];

  const int tid = threadIdx.x, cg = tid % G::CG, rg = tid / G::CG;
  // 1-D grid: block = bh * C1 + c (any number of planes)
  const int64_t bh = blockIdx.x / C1, c = blockIdx.x - bh * C1;
  const int64_t b = bh / H, h = bh - b * H;
  const T* kp = K + b * k_sb + h * k_sh + 8 * cg;
  const T* vp = V + b * v_sb + h * v_sh + 8 * cg;
  u8* vt = V8T + bh * D * N_pad;
  const int64_t r_begin = c * R1;
  // the plane's last block also covers the pure pad rows up to N_pad
  const int64_t r_end = (c == C1 - 1 || r_begin + R1 > N_pad) ? N_pad : r_begin + R1;
  const bool k_sums = (smooth_k && VMODE != V_CENTERED) || VMODE == K_ONLY;
  if (VMODE == K_ONLY && r_begin >= N) {   // nothing but pad rows: zero partials
    if (tid < D) part[(bh * C1 + c) * D + tid] = 0.0;
    return;
  }

  // V's sequence mean (V_CENTERED): every block of the plane reduces the same partials in the
  // same order, so all of them subtract the same bits.
  float vmu[8];
  if (VMODE == V_CENTERED) {
    if (tid < D) {
      double sum = 0.0;
      for (int64_t cc = 0; cc < C1; ++cc) sum += vpart[(bh * C1 + cc) * D + tid];
      const float m = (float)(sum / (double)N);
      vmu_s[tid] = m;
      if (c == 0) VMEAN[bh * D + tid] = m;
    }
    __syncthreads();
#pragma unroll
    for (int e = 0; e < 8; ++e) vmu[e] = vmu_s[8 * cg + e];
  }

  double ks[8], vs[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) ks[i] = vs[i] = 0.0;
  float sv_max = 0.0f;

  for (int64_t n0 = r_begin; n0 < r_end; n0 += STEP) {
    u32x4 vw[8], kw[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int64_t n = n0 + 8 * rg + i;
      const bool live = n < N;
      vw[i] = (live && VMODE != K_ONLY) ? *(const u32x4*)(vp + n * v_sr) : (u32x4){0u, 0u, 0u, 0u};
      kw[i] = (live && k_sums) ? *(const u32x4*)(kp + n * k_sr) : (u32x4){0u, 0u, 0u, 0u};
    }
    if (k_sums) {
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        float f[8];
        unpack8<T>(kw[i], f);
#pragma unroll
        for (int e = 0; e < 8; ++e) ks[e] += (double)f[e];
      }
    }
    if (VMODE == V_SUMS) {
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        float f[8];
        unpack8<T>(vw[i], f);
#pragma unroll
        for (int e = 0; e < 8; ++e) vs[e] += (double)f[e];
      }
      continue;
    }
    if (VMODE == K_ONLY) continue;
    // V: per-row scale and e4m3 bytes. col_lo/col_hi[e] collect tokens 0..3 / 4..7 of column e.
    uint32_t col_lo[8], col_hi[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) col_lo[e] = col_hi[e] = 0u;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int64_t n = n0 + 8 * rg + i;
      const bool live = n < N;
      float f[8];
      unpack8<T>(vw[i], f);
      if (VMODE == V_CENTERED) {
        // centred before the absmax; pad rows stay zero
#pragma unroll
        for (int e = 0; e < 8; ++e) f[e] = live ? f[e] - vmu[e] : 0.0f;
      }
      float vmax = 0.0f;
#pragma unroll
      for (int e = 0; e < 8; ++e) vmax = fmaxf(vmax, fabsf(f[e]));
      vmax = maxg<G::CG>(vmax);
      // sv = max(RN(vmax / 448), 1e-12); the row's quotients RN(v / sv) come from one correctly
      // rounded reciprocal of sv (div_by: bit-identical to a division per element)
      const float sv = fmaxf(div_by(vmax, P_SCALE, RCP_P_SCALE), SCALE_FLOOR);
      const float rsv = __fdiv_rn(1.0f, sv);
      if (cg == 0 && n < N_pad) SV[bh * N_pad + n] = live ? sv : 0.0f;
      if (live) sv_max = fmaxf(sv_max, sv);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const uint32_t byte = fp8x2(fminf(div_by(f[e], sv, rsv), P_SCALE), 0.0f) & 0xffu;
        if (i < 4)
          col_lo[e] |= byte << (8 * i);
        else
          col_hi[e] |= byte << (8 * (i - 4));
      }
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int d = 8 * cg + e;
      const int pos = rg ^ cg;  // d >> 3 == cg
      *(u32x2*)(tile + d * VT_STRIDE + 8 * pos) = (u32x2){col_lo[e], col_hi[e]};
    }
    __syncthreads();
    {
      // PT/D threads per row d, 64 tokens (4 x 16 bytes) each
      constexpr int TPD = PT / D;
      const int d = tid / TPD, part = tid % TPD, dx = d >> 3;
      const int64_t nb = n0 + 64 * part;
      if (nb < N_pad) {
#pragma unroll
        for (int m = 0; m < 4; ++m) {
          const int r0 = 8 * part + 2 * m;  // token chunks r0, r0+1 (8 tokens each)
          const int p0 = r0 ^ dx;
          u32x4 x = *(const u32x4*)(tile + d * VT_STRIDE + 8 * (p0 & ~1));
          if (p0 & 1) x = (u32x4){x.z, x.w, x.x, x.y};
          *(u32x4*)(vt + (int64_t)d * N_pad + nb + 16 * m) = x;
        }
      }
    }
    __syncthreads();
  }

  // fp64 mean partials: reduce the RG row groups in a fixed order.
  static_assert(RG * D * sizeof(double) <= sizeof(tile), "reduction buffer");
  double* red = (double*)tile;  // RG x D doubles = 16 KB
  if (k_sums) {
#pragma unroll
    for (int e = 0; e < 8; ++e) red[rg * D + 8 * cg + e] = ks[e];
    __syncthreads();
    if (tid < D) {
      double s = 0.0;
#pragma unroll
      for (int r = 0; r < RG; ++r) s += red[r * D + tid];
      part[(bh * C1 + c) * D + tid] = s;
    }
    __syncthreads();
  }
  if (VMODE == V_SUMS) {
#pragma unroll
    for (int e = 0; e < 8; ++e) red[rg * D + 8 * cg + e] = vs[e];
    __syncthreads();
    if (tid < D) {
      double s = 0.0;
#pragma unroll
      for (int r = 0; r < RG; ++r) s += red[r * D + tid];
      vpart[(bh * C1 + c) * D + tid] = s;
    }
    return;   // V is quantized by the V_CENTERED launch
  }
  if (VMODE == K_ONLY) return;
  // block max of sv over live rows
  float m = sv_max;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
  if ((tid & 63) == 0) wmax[tid >> 6] = m;
  __syncthreads();
  if (tid == 0) smax[bh * C1 + c] = fmaxf(fmaxf(wmax[0], wmax[1]), fmaxf(wmax[2], wmax[3]));
}

// ---------------------------------------------------------------------------------------------
// Quant pass. grid (C2, BH), block 256. Thread (cg, rg) handles row base+rg+16i, columns 8cg..+7.
// ---------------------------------------------------------------------------------------------
template <typename T, bool KINT8, int D>
__global__ __launch_bounds__(PT) __attribute__((amdgpu_waves_per_eu(QUANT_BLOCKS_PER_CU))) void k_quant_kernel(
    const T* __restrict__ K, u8* __restrict__ K8, float* __restrict__ SK, float* __restrict__ SV,
    const double* __restrict__ part, const float* __restrict__ smax, float* __restrict__ MEAN,
    float* __restrict__ S_out, float* __restrict__ KC, int64_t H, int64_t N, int64_t N_pad,
    int64_t R2, int64_t C2, int64_t C1,
    int64_t k_sb, int64_t k_sh, int64_t k_sr, int smooth_k, int fold) {
  using G = Geo<D>;
  constexpr int RG = G::RG;
  __shared__ float mu_s[D];
  __shared__ float s_fold;

  const int tid = threadIdx.x, cg = tid % G::CG, rg = tid / G::CG;
  // 1-D grid: block = bh * C2 + c2 (any number of planes)
  const int64_t bh = blockIdx.x / C2, c2 = blockIdx.x - bh * C2;
  const int64_t b = bh / H, h = bh - b * H;

  if (tid < D) {
    float mu = 0.0f;
    if (smooth_k) {
      double s = 0.0;
      for (int64_t c = 0; c < C1; ++c) s += part[(bh * C1 + c) * D + tid];
      mu = (float)(s / (double)N);
      if (MEAN != nullptr && c2 == 0) MEAN[bh * D + tid] = mu;
    }
    mu_s[tid] = mu;
  } else if (tid < D + 64) {
    const int l = tid - D;
    float m = 1.0f;
    for (int64_t c = l; c < C1; c += 64) m = fmaxf(m, smax[bh * C1 + c]);
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
    if (l == 0) {
      s_fold = m;
      if (c2 == 0) S_out[bh] = m;
    }
  }
  __syncthreads();

  float mu[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) mu[e] = mu_s[8 * cg + e];
  const float S = s_fold;
  const T* kp = K + b * k_sb + h * k_sh + 8 * cg;
  const int64_t r_begin = c2 * R2;
  const int64_t r_end = (r_begin + R2 < N_pad) ? r_begin + R2 : N_pad;

  for (int64_t n0 = r_begin; n0 < r_end; n0 += 64) {
    // 64 rows per step: rows n0 + rg + RG*i
    u32x4 kw[64 / RG];
#pragma unroll
    for (int i = 0; i < 64 / RG; ++i) {
      const int64_t n = n0 + rg + RG * i;
      kw[i] = (n < N) ? *(const u32x4*)(kp + n * k_sr) : (u32x4){0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int i = 0; i < 64 / RG; ++i) {
      const int64_t n = n0 + rg + RG * i;
      const bool live = n < N;
      float kc[8];
      unpack8<T>(kw[i], kc);
      float kmax = 0.0f;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        kc[e] = live ? (smooth_k ? kc[e] - mu[e] : kc[e]) : 0.0f;
        kmax = fmaxf(kmax, fabsf(kc[e]));
      }
      kmax = maxg<G::CG>(kmax);
      // sk = max(RN(kmax / 127 or 448), 1e-12); quotients RN(kc / sk) through one reciprocal
      const float sk = fmaxf(KINT8 ? div_by(kmax, I8_MAX, RCP_I8_MAX)
                                   : div_by(kmax, P_SCALE, RCP_P_SCALE), SCALE_FLOOR);
      const float rsk = __fdiv_rn(1.0f, sk);
      if (n < r_end) {
        u32x2 word;
        if (KINT8) {
          float x[8];
#pragma unroll
          for (int e = 0; e < 8; ++e) x[e] = div_by(kc[e], sk, rsk);
          word = (u32x2){i8x4(x[0], x[1], x[2], x[3]), i8x4(x[4], x[5], x[6], x[7])};
        } else {
          float x[8];
#pragma unroll
          for (int e = 0; e < 8; ++e) x[e] = fminf(div_by(kc[e], sk, rsk), P_SCALE);
          word = (u32x2){fp8x4(x[0], x[1], x[2], x[3]), fp8x4(x[4], x[5], x[6], x[7])};
        }
        *(u32x2*)(K8 + (bh * N_pad + n) * D + 8 * cg) = word;
        // The main loop's per-key constants of 64-key block n/64 (KC, optional): SK and
        // RN(SV'*448), 64 floats each.
        float* kc = KC ? KC + (bh * (N_pad / 64) + n / 64) * 128 + (n & 63) : nullptr;
        if (cg == 0) {
          const float ske = live ? sk : 1.0f;
          SK[bh * N_pad + n] = ske;
          if (kc) kc[0] = ske;
        }
        if (cg == 1) {
          const float sv = SV[bh * N_pad + n];
          const float svp = fold ? __fdiv_rn(sv, S) : sv;
          if (fold) SV[bh * N_pad + n] = svp;
          if (kc) kc[64] = svp * P_SCALE;
        }
      }
    }
  }
}

template <typename T, int D>
static hipError_t launch_prologue_t(const PrologueArgs& a, hipStream_t stream) {
  const int64_t BH = a.B * a.H;
  const PrologueGeom g = prologue_geom(BH, a.N, a.N_pad, Geo<D>::STEP, a.cus);
  // region offsets as sized for head_dim 128 (prologue_workspace_bytes)
  const size_t part_bytes = part_region_bytes(BH, prologue_geom(BH, a.N, a.N_pad));
  double* part = (double*)a.workspace;
  double* vpart = (double*)((char*)a.workspace + part_bytes);
  float* smax = (float*)((char*)a.workspace + 2 * part_bytes);
  const dim3 grid1((unsigned)(g.C1 * BH));
  if (a.smooth_v) {
    // V's mean first (with K's partials), then V - mean quantized
    hipLaunchKernelGGL((kv_stats_kernel<T, V_SUMS, D>), grid1, dim3(PT), 0, stream, (const T*)a.k,
                       (const T*)a.v, (u8*)a.v8t, a.sv, part, vpart, a.vmean, smax, a.H, a.N,
                       a.N_pad, g.R1, g.C1, a.k_sb, a.k_sh, a.k_sr, a.v_sb, a.v_sh, a.v_sr,
                       a.smooth_k);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL((kv_stats_kernel<T, V_CENTERED, D>), grid1, dim3(PT), 0, stream,
                       (const T*)a.k, (const T*)a.v, (u8*)a.v8t, a.sv, part, vpart, a.vmean, smax,
                       a.H, a.N, a.N_pad, g.R1, g.C1, a.k_sb, a.k_sh, a.k_sr, a.v_sb, a.v_sh,
                       a.v_sr, a.smooth_k);
  } else {
    hipLaunchKernelGGL((kv_stats_kernel<T, V_QUANT, D>), grid1, dim3(PT), 0, stream, (const T*)a.k,
                       (const T*)a.v, (u8*)a.v8t, a.sv, part, vpart, a.vmean, smax, a.H, a.N,
                       a.N_pad, g.R1, g.C1, a.k_sb, a.k_sh, a.k_sr, a.v_sb, a.v_sh, a.v_sr,
                       a.smooth_k);
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  const dim3 grid2((unsigned)(g.C2 * BH));
  if (a.k_int8)
    hipLaunchKernelGGL((k_quant_kernel<T, true, D>), grid2, dim3(PT), 0,
                       stream, (const T*)a.k, (u8*)a.k8, a.sk, a.sv, part, smax, a.mean, a.s, a.kconst, a.H,
                       a.N, a.N_pad, g.R2, g.C2, g.C1, a.k_sb, a.k_sh, a.k_sr, a.smooth_k, a.fold);
  else
    hipLaunchKernelGGL((k_quant_kernel<T, false, D>), grid2, dim3(PT), 0,
                       stream, (const T*)a.k, (u8*)a.k8, a.sk, a.sv, part, smax, a.mean, a.s, a.kconst, a.H,
                       a.N, a.N_pad, g.R2, g.C2, g.C1, a.k_sb, a.k_sh, a.k_sr, a.smooth_k, a.fold);
  return hipGetLastError();
}

// MEAN from the stats pass's K partials: the reduction of k_quant_kernel (same order, same
// rounding), one block of D threads per plane.
template <int D>
__global__ __launch_bounds__(D) void mean_reduce_kernel(const double* __restrict__ part,
                                                        float* __restrict__ MEAN, int64_t N,
                                                        int64_t C1) {
  const int64_t bh = blockIdx.x;
  const int tid = threadIdx.x;
  double s = 0.0;
  for (int64_t c = 0; c < C1; ++c) s += part[(bh * C1 + c) * D + tid];
  MEAN[bh * D + tid] = (float)(s / (double)N);
}

template <typename T, int D>
static hipError_t launch_kseq_mean_t(const PrologueArgs& a, hipStream_t stream) {
  const int64_t BH = a.B * a.H;
  const PrologueGeom g = prologue_geom(BH, a.N, a.N_pad, Geo<D>::STEP, a.cus);
  double* part = (double*)a.workspace;
  hipLaunchKernelGGL((kv_stats_kernel<T, K_ONLY, D>), dim3((unsigned)(g.C1 * BH)), dim3(PT), 0,
                     stream, (const T*)a.k, (const T*)a.k, nullptr, nullptr, part, nullptr, nullptr,
                     nullptr, a.H, a.N, a.N_pad, g.R1, g.C1, a.k_sb, a.k_sh, a.k_sr, a.k_sb,
                     a.k_sh, a.k_sr, 1);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL((mean_reduce_kernel<D>), dim3((unsigned)BH), dim3(D), 0, stream, part, a.mean,
                     a.N, g.C1);
  return hipGetLastError();
}

hipError_t launch_kseq_mean(const PrologueArgs& a, hipStream_t stream) {
  if (a.D == 64)
    return a.dtype == 1 ? launch_kseq_mean_t<bf16, 64>(a, stream)
                        : launch_kseq_mean_t<f16, 64>(a, stream);
  return a.dtype == 1 ? launch_kseq_mean_t<bf16, 128>(a, stream)
                      : launch_kseq_mean_t<f16, 128>(a, stream);
}

hipError_t launch_prologue(const PrologueArgs& a, hipStream_t stream) {
  if (a.D == 64)
    return a.dtype == 1 ? launch_prologue_t<bf16, 64>(a, stream)
                        : launch_prologue_t<f16, 64>(a, stream);
  return a.dtype == 1 ? launch_prologue_t<bf16, 128>(a, stream)
                      : launch_prologue_t<f16, 128>(a, stream);
}

}  // namespace sage
