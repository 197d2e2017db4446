// The main loop, software-pipelined inside each wave: three waves per SIMD, each issuing its own
// matrix work between its own softmax instructions.
//
// Scheme, layouts and per-score arithmetic are those of attn_fwd.hip (the reference's
// kernels/hip/sk1_t6i.hip:84-299 and sk1_t4a1s.hip): transposed scores S^T = K . Q^T so that a
// lane holds one query, per-key constants as DPP row broadcasts, the exact running max in x units,
// P folded into e4m3 as the P.V operand. Every score, row sum and accumulator update is the same
// operation on the same values as in attn_fwd.hip, so the two kernels give the same bits; what
// differs is when each wave issues its MFMAs.
//
// Why: the softmax is VALU work and on gfx950 one wave issues at most one VALU instruction every
// ~5-6 cycles, while three or four waves issuing together reach ~2-3 cycles per instruction
// (measured: the per-block softmax costs its SIMD ~1250 cycles with one wave issuing, ~800 with
// three). A wave that waits for its own S^T tile or P.V does not issue, so here no wave waits for
// its matrix work: in iteration j a wave
//   * issues P.V of block j-1 (its P and alpha were finished in iteration j-1),
//   * runs the softmax of block j on S^T(j), which it computed in iteration j-1,
//   * issues S^T(j+1) = K(j+1) . Q^T tile by tile, each tile as soon as the softmax has consumed
//     the scores of the tile whose registers it reuses.
// The matrix core then runs behind the softmax of the same wave and of the two other waves of the
// SIMD, which belong to other blocks and drift freely against it.
//
// Block: 4 waves x 32 queries (128 queries of one plane), one wave per SIMD; three blocks per CU
// at head_dim 128 (168 VGPRs, 3 x 50 KB LDS), four at head_dim 64. K tiles, V^T tiles and the
// per-key constants go global -> LDS directly (global_load_lds) into a ring of three buffers: the
// tiles of block j+2 are requested in iteration j, after the iteration's barrier, into the buffer
// block j-1 used (whose V^T tile every wave read before that barrier).
//
// Per-key constants are read from two rows per 64-key block with strides, so the same kernel reads
// the reference's SK and SV' arrays (W = RN(SV' * 448) formed on load) or the prologue's KCONST
// layout (W already formed, multiplied by 1).
//
// The SPLIT form (non-causal head_dim 64, for grids that leave compute units idle) is described
// at the kernel: 64 queries per block, the key blocks shared out between two wave pairs.
#include "attn_common.h"
#include "sage_launch.h"

namespace sage {

// Per-key constants of one 64-key block in LDS: SK and the fold source (SV' or RN(SV' * 448)).
struct KeyRows {
  float sk[BK];
  float w[BK];
};

template <int D>
struct __attribute__((aligned(16))) PlBuf {
  u8 k[BK * D];
  u8 v[D * BK];
  KeyRows c;
};

// Waves per SIMD the pipelined kernel's register budget is sized for. The key-split form (head_dim
// 64) holds two staging rings and the block-max exchange, 52 KB of LDS, so three of its blocks
// fit a CU.
constexpr int pl_waves(int D, bool split = false) { return split ? 3 : (D == 64 ? 4 : 3); }

// SPLIT (non-causal, head_dim 64; the key-split form for grids that leave compute units idle): a
// block of 64 queries whose two wave pairs (key groups) run the same queries on alternate 64-key
// blocks -- group 0 the even blocks, group 1 the odd ones -- each pair with its own staging ring.
// Each iteration both groups publish their block's row maxima in LDS before the loop's barrier
// and read the other's after it, so both know the running max of the whole sequence up to their
// block: block b's probabilities are shifted by exactly the max over blocks 0..b, the shift the
// sequential loop uses, and P is bit for bit the other kernels'. Each group keeps its own row
// sum and O^T relative to its last shift; at the end group 1 hands them to group 0 through LDS,
// which rescales both to the larger shift and writes the output. Only the fp32 sums differ from
// the sequential loop's (rescaled per group, then merged): rounding-level output differences.
template <typename T, bool QK_INT8, bool CAUSAL, int D, bool SPLIT = false>
__global__ __launch_bounds__(AT) __attribute__((amdgpu_waves_per_eu(pl_waves(D, SPLIT), pl_waves(D, SPLIT)))) void attn_fwd_pl_kernel(
    const T* __restrict__ Q, const u8* __restrict__ K8, const float* __restrict__ SKr,
    int64_t sk_plane, int64_t sk_block, const float* __restrict__ Wr, int64_t w_plane,
    int64_t w_block, float w_mul, const u8* __restrict__ V8T, const float* __restrict__ Sfold,
    T* __restrict__ O, int64_t q_sb, int64_t q_sh, int64_t q_sr, int64_t o_sb, int64_t o_sh,
    int64_t o_sr, int H, int H_kv, int G, int N, int Nk, int Nk_pad, int num_qt, int xcd_span,
    float sm_scale, float* __restrict__ LSE, const float* __restrict__ KMEAN,
    const float* __restrict__ VMEAN) {
  static_assert(!(SPLIT && (CAUSAL || D != 64)), "the key split serves non-causal head_dim 64");
  __shared__ PlBuf<D> sBall[SPLIT ? 6 : 3];
  // SPLIT: the per-iteration exchange of block maxima (two slots, 4 waves x 32 queries). The
  // block's LDS, 53248 bytes, is 26 units of 2 KB: three blocks fit a CU's 160 KB (one more
  // 2 KB unit each would leave room for two).
  __shared__ float xch[SPLIT ? 2 : 1][SPLIT ? 4 * 32 : 1];
  constexpr int NDT = D / 32;   // 32-channel output tiles per wave
  // 1 KB K and V^T requests per wave and block (each): a tile of D/16 KB over the 4 waves, or
  // over the 2 waves of a key group
  constexpr int NKV = (SPLIT ? 2 : 1) * D / 64;
  constexpr int QB = SPLIT ? 64 : BM;          // queries per block

  // ---- which (plane, q-tile) this block runs: XCD-contiguous planes, longest causal tiles first
  int id = blockIdx.x;
  if (id < xcd_span) id = (id & 7) * (xcd_span >> 3) + (id >> 3);
  const int bh = id / num_qt;
  int qt = id - bh * num_qt;
  if (CAUSAL) qt = num_qt - 1 - qt;
  const int b = bh / H, hd = bh - b * H;
  const int kvp = b * H_kv + hd / G;   // the K/V plane this query plane reads (GQA: G heads share it)

  const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l32 = lane & 31, hh = lane >> 5;
  // SPLIT: wave w runs query slot w & 1 of key group w >> 1 (the waves of a group: 2 of them,
  // staging a tile together); otherwise one group of 4 waves, query slot w
  const int kg = SPLIT ? (w >> 1) : 0;
  const int ws = SPLIT ? (w & 1) : w;            // query slot, and staging index within the group
  const int q0 = qt * QB + ws * 32;
  const int qrow = q0 + l32;
  PlBuf<D>* sB = sBall + 3 * kg;

  const int n_blocks = Nk_pad / BK;
  // this group's key blocks: iteration j runs block KS * j + kg (SPLIT: kg + 2j, the even or
  // the odd blocks), n_g of them
  constexpr int KS = SPLIT ? 2 : 1;
  const int n_g = SPLIT ? (n_blocks + 1 - kg) >> 1 : n_blocks;
  const int j_end = CAUSAL ? min(n_blocks, (qt * BM + BM - 1) / BK + 1)
                           : (SPLIT ? (n_blocks + 1) >> 1 : n_g);
  // blocks this wave computes: 0 .. w_end-1 (the rest of the j_end iterations it only stages)
  const int w_end = CAUSAL ? min(j_end, (q0 + 31) / BK + 1) : n_g;

  const u8* Kb = K8 + (int64_t)kvp * Nk_pad * D + (int64_t)kg * BK * D;
  const u8* Vb = V8T + (int64_t)kvp * D * Nk_pad + (int64_t)kg * BK;
  // wave (slot) 0 of the group stages the SK row of each block, slot 1 the W row
  const float* Cb = ((ws == 0) ? SKr + (int64_t)kvp * sk_plane : Wr + (int64_t)kvp * w_plane)
                    + (int64_t)kg * ((ws == 0) ? sk_block : w_block);
  const uint32_t c_blk = (uint32_t)(4 * KS * ((ws == 0) ? sk_block : w_block));

  // ---- staging: per block every wave issues NKV KB of K and NKV KB of V^T; waves 0 and 1 also
  // 256 bytes of constants (SK, W). Layouts as in attn_fwd.hip.
  uint32_t k_off[NKV], v_off[NKV];
#pragma unroll
  for (int i = 0; i < NKV; ++i) {
    const int I = NKV * ws + i;
    const int krow = (1024 / D) * I + lane / (D / 16), kpos = lane % (D / 16);
    k_off[i] = (uint32_t)(krow * D + 16 * (kpos ^ kswz<D>(krow)));
    const int d = 16 * I + (lane >> 2), vpos = lane & 3;
    v_off[i] = (uint32_t)(d * Nk_pad + 16 * (vpos ^ vswz(d)));
  }
  const uint32_t c_off = (uint32_t)(4 * lane);
  auto dma = [&](int j, PlBuf<D>& buf) {
    const u8* kblk = Kb + (size_t)(KS * BK * D) * (uint32_t)j;
    const u8* vblk = Vb + (size_t)(KS * BK) * (uint32_t)j;
    const uint32_t kl = lds_addr(buf.k) + 1024 * NKV * ws, vl = lds_addr(buf.v) + 1024 * NKV * ws;
#pragma unroll
    for (int i = 0; i < NKV; ++i) dma16(kblk, k_off[i], kl + 1024 * i);
#pragma unroll
    for (int i = 0; i < NKV; ++i) dma16(vblk, v_off[i], vl + 1024 * i);
    if (ws < 2) dma4(Cb, c_off + c_blk * (uint32_t)j, lds_addr(ws == 0 ? buf.c.sk : buf.c.w));
  };

  if (!SPLIT || n_g > 0) dma(0, sB[0]);
  if ((SPLIT ? n_g : j_end) > 1) dma(1, sB[1]);

  // ---- Q: per-row quantization straight into MFMA fragments ----
  QFrag<D> qf;
  float sq, cq;
  float qmu = 0.0f;   // q . mu for the logsumexp's smooth_k correction (when asked)
  quant_q_row<T, QK_INT8, D>(Q + b * q_sb + hd * q_sh + (int64_t)qrow * q_sr, qrow < N, hh,
                             sm_scale, qf, sq, cq,
                             (LSE && KMEAN) ? KMEAN + (int64_t)kvp * D : nullptr, &qmu);
  (void)sq;
  const float Sb = Sfold[kvp];

  f32x16 acc[NDT];
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[dt][r] = 0.0f;
  float m_x = -INFINITY;     // running max of x = (Q8.K8)*SK for this lane's query
  float mc = -INFINITY;      // RN(c_q * m_x), the exp2 shift in use
  float l_i = 0.0f;
  float r_all = -INFINITY;   // SPLIT: the running max over every block both groups have run
  // P of the block whose P.V is issued next: zero before the first block and after the wave's
  // last, so that the P.V at the top of every iteration is unconditional (it adds zero there)
  i32x8 pb;
#pragma unroll
  for (int i = 0; i < 8; ++i) pb[i] = 0;

  const int krow0 = kappa(0, l32), krow1 = kappa(1, l32);
  const int ksw0 = kswz<D>(krow0), ksw1 = kswz<D>(krow1);
  const int vrow = l32;               // + 32 dt
  const int vsw = vswz(vrow);         // vswz(32dt + r) == vswz(r)

  // O^T += V^T . P^T for the block whose V^T tile is in `vbuf` (acc was rescaled by that block's
  // alpha when the alpha was formed)
  auto pv = [&](const u8* vbuf) {
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) {
      const u8* vb = vbuf + (32 * dt + vrow) * BK;
      const i32x4 lo = *(const i32x4*)(vb + 16 * ((2 * hh) ^ vsw));
      const i32x4 hi = *(const i32x4*)(vb + 16 * ((2 * hh + 1) ^ vsw));
      const i32x8 vf = (i32x8){lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
      acc[dt] = mfma_f8(vf, pb, acc[dt]);
    }
    // The products are pinned here: MFMAs touch no memory, and without the pins the compiler
    // sinks them past the barrier into the softmax that follows (or out of the iteration).
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) keep_live(acc[dt]);
  };

  // The first iteration's P.V reads buffer 2's V^T tile before block 2 lands there, with P = 0:
  // zero it, so that it adds exactly zero (uninitialized LDS may hold NaN patterns). A key group
  // of the split with fewer than two blocks also reads buffers it never loads: zero those too.
  constexpr int GT = SPLIT ? AT / 2 : AT;      // threads of a key group
  constexpr int ZB = D * BK / GT;              // bytes of the tile per thread: 16 .. 64
  const int gtid = SPLIT ? (tid & (GT - 1)) : tid;
  for (int zb = SPLIT ? min(n_g, 2) : 2; zb < 3; ++zb) {
#pragma unroll
    for (int i = 0; i < ZB / 16; ++i)
      *(u32x4*)(sB[zb].v + ZB * gtid + 16 * i) = (u32x4){0u, 0u, 0u, 0u};
  }
  __builtin_amdgcn_s_waitcnt(0);    // blocks 0 and 1 landed (once per block of queries)
  __syncthreads();

  f32x16 st[2];   // S^T of the block whose softmax comes next
  st[0] = qk_tile<QK_INT8, D>(sB[0].k, qf, krow0, ksw0, hh);
  st[1] = qk_tile<QK_INT8, D>(sB[0].k, qf, krow1, ksw1, hh);
  keep_live(st[0]);
  keep_live(st[1]);
  mfma_result_fence();   // the first softmax reads these right away

  // Iteration j (j = 0 .. j_end; the last only drains). Buffer j % 3 holds block j's constants
  // (read now) and V^T tile (read in iteration j+1); buffer (j+2) % 3 holds block j-1's V^T tile
  // (read at the top, before the barrier) and then receives block j+2's tiles; buffer (j+1) % 3
  // holds block j+1's K tile. One loop body, buffers chosen at run time: with the body unrolled
  // by buffer the compiler moved accumulators between register ranges at the seams, and such a
  // copy can read an MFMA result before the MFMA has written it.
  int pc = 0;   // j % 3
  // block j's per-key constants, read from LDS one iteration ahead (block 0's here)
  float ksk0, ksk1, kw0, kw1;
  auto load_consts = [&](const PlBuf<D>& buf) {
    const int c = 32 * hh + (lane & 15);
    ksk0 = buf.c.sk[c];
    ksk1 = buf.c.sk[c + 16];
    kw0 = buf.c.w[c];
    kw1 = buf.c.w[c + 16];
  };
  load_consts(sB[0]);
  for (int j = 0; j <= j_end; ++j) {
    const int pm = pc == 0 ? 2 : pc - 1, pn = pc == 2 ? 0 : pc + 1;
    PlBuf<D>& bcur = sB[pc];
    PlBuf<D>& bprev = sB[pm];
    PlBuf<D>& bnext = sB[pn];
    const bool compute = j < w_end;
    // Each section is a scheduling region of its own: the compiler neither hoists one
    // iteration's LDS operand reads into the previous one nor mixes the sections' live ranges.
    __builtin_amdgcn_sched_barrier(0);
    // P.V of block j-1 (at j == 0 and after the wave's last block, P is zero); at j == w_end
    // this drains the wave's pipeline
    pv(bprev.v);
    __builtin_amdgcn_sched_barrier(0);
    if (j == j_end) break;
    if (!compute) {
#pragma unroll
      for (int i = 0; i < 8; ++i) pb[i] = 0;
    }
    // the softmax's first half on S^T(j): scores, masks, the running max and the block's shift
    BlockShift sh = {0.0f, 1.0f};
    float w0 = 0.0f, w1 = 0.0f;
    float mx = -INFINITY;   // SPLIT: the row max of this group's block (-inf without one)
    if (compute) {
      w0 = kw0 * w_mul;
      w1 = kw1 * w_mul;
      if constexpr (SPLIT) {
        mx = block_max<QK_INT8, false>(st, ksk0, ksk1, KS * j + kg, q0, qrow, Nk, hh);
      } else {
        sh = scores_block<QK_INT8, CAUSAL>(st, ksk0, ksk1, j, q0, qrow, Nk, hh, cq, m_x, mc);
        // acc *= alpha before block j's P.V (issued next iteration); P.V of block j-1 was
        // issued above, a whole scores pass ago
        rescale_acc(acc, sh.alpha);
      }
    }
    if constexpr (SPLIT) {
      if (hh == 0) xch[j & 1][32 * w + l32] = mx;
    }
    // This wave's requests for block j+1 have landed; after the barrier every wave's have, and
    // every wave has read block j-1's V^T tile, so its buffer takes block j+2. (SPLIT: and both
    // groups' block maxima of this iteration are in LDS.)
    __builtin_amdgcn_sched_barrier(0);
    asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
    // SPLIT: the other group's block max (wave w ^ 2 runs the same queries), read before the
    // staging requests are issued so that they cover its latency. The slot is written again two
    // iterations on, after the partner has passed the next barrier.
    float om = -INFINITY;
    if constexpr (SPLIT) om = xch[j & 1][32 * (w ^ 2) + l32];
    if (j + 2 < (SPLIT ? n_g : j_end)) dma(j + 2, bprev);
    if constexpr (SPLIT) {
      // blocks 2j (group 0) and 2j+1 (group 1) are now both known. rb: the max over blocks
      // 0..b for this group's block b; r_all: over every block so far.
      float rb;
      if (kg == 0) {
        rb = fmaxf(r_all, mx);
        r_all = fmaxf(rb, om);
      } else {
        rb = fmaxf(fmaxf(r_all, om), mx);
        r_all = rb;
      }
      if (compute) {
        // scores_block's update with the sequence's max: this group's O^T and row sum are
        // relative to the shift of its previous block (m_x, mc)
        const float mcb = shift_of(rb, cq);
        sh.alpha = (rb != m_x) ? __builtin_amdgcn_exp2f(mc - mcb) : 1.0f;
        sh.mc = mcb;
        m_x = rb;
        mc = mcb;
        rescale_acc(acc, sh.alpha);
      }
    }
    // the second half, tile by tile; S^T(j+1) tile t is issued into the registers of the scores
    // of tile t as soon as they are consumed
    if (compute) {
      float ps[4];
      probs_tile<0>(st, w0, cq, sh.mc, ps, pb);
      st[0] = qk_tile<QK_INT8, D>(bnext.k, qf, krow0, ksw0, hh);
      keep_live(st[0]);
      __builtin_amdgcn_sched_barrier(0);
      probs_tile<1>(st, w1, cq, sh.mc, ps, pb);
      st[1] = qk_tile<QK_INT8, D>(bnext.k, qf, krow1, ksw1, hh);
      keep_live(st[1]);
      asm volatile("" ::"v"(pb));
      __builtin_amdgcn_sched_barrier(0);
      const float psum = sum_halves((ps[0] + ps[1]) + (ps[2] + ps[3]));
      l_i = __builtin_fmaf(l_i, sh.alpha, psum);
      // block j+1's constants: in buffer (j+1) % 3 since this iteration's barrier
      load_consts(bnext);
    }
    pc = pn;
  }
  // acc is read below only inside the divergent `qrow < N` branch; keep the loop's MFMAs out
  // of it (an MFMA under a partial EXEC mask loses the inactive lanes' operand rows).
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt) keep_live(acc[dt]);
  mfma_result_fence();

  if constexpr (SPLIT) {
    // Merge the key halves: group 1 parks O^T, mc and l of each lane in LDS (the staging ring is
    // free once every wave has passed the barrier), group 0 takes M = max(mc0, mc1) and
    // rescales both halves to it: l = l0 * 2^(mc0 - M) + l1 * 2^(mc1 - M), the same for O^T.
    // A half without keys has mc = -inf, so its factor is 0.
    constexpr int NE = 16 * NDT + 2;
    float* park = (float*)sBall + ws * (NE * 64);
    asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
    if (kg == 1) {
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
        for (int r = 0; r < 16; ++r) park[(16 * dt + r) * 64 + lane] = acc[dt][r];
      park[(16 * NDT) * 64 + lane] = mc;
      park[(16 * NDT + 1) * 64 + lane] = l_i;
    }
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    if (kg == 0) {
      const float mc1 = park[(16 * NDT) * 64 + lane];
      const float l1 = park[(16 * NDT + 1) * 64 + lane];
      const float M = fmaxf(mc, mc1);
      const float a0 = (mc == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(mc - M);
      const float a1 = (mc1 == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(mc1 - M);
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
        for (int r = 0; r < 16; ++r)
          acc[dt][r] = __builtin_fmaf(acc[dt][r], a0, park[(16 * dt + r) * 64 + lane] * a1);
      l_i = __builtin_fmaf(l_i, a0, l1 * a1);
      mc = M;
    }
  }

  // ---------- epilogue: O = acc * S / (l * 448) (+ V's mean with smooth_v, one fma) ----------
  if (qrow < N && kg == 0) {
    if (LSE && hh == 0) LSE[(int64_t)bh * N + qrow] = row_lse(mc, l_i, sm_scale, qmu);
    const float inv = (l_i > 0.0f) ? __fdiv_rn(Sb, l_i * P_SCALE) : 0.0f;
    T* op = O + b * o_sb + hd * o_sh + (int64_t)qrow * o_sr;
    const float* vmp = VMEAN ? VMEAN + (int64_t)kvp * D : nullptr;
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int d = 32 * dt + 8 * g + 4 * hh;
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

template <typename T, bool QK_INT8, bool CAUSAL, int D, bool SPLIT = false>
static void launch_pl_d(const AttnArgs& a, hipStream_t stream) {
  const int BH = (int)(a.B * a.H);
  const int num_qt = (int)((a.N + (SPLIT ? 64 : BM) - 1) / (SPLIT ? 64 : BM));
  const int total = num_qt * BH;
  const int span = (total / 8) * 8;
  // per-key constant rows: the reference's SK / SV' arrays, or the prologue's KCONST layout
  const bool kc = a.kconst != nullptr;
  const float* skr = kc ? a.kconst : a.sk;
  const float* wr = kc ? a.kconst + BK : a.svp;
  const int64_t plane = kc ? 2 * a.N_kv_pad : a.N_kv_pad, blk = kc ? 2 * BK : BK;
  hipLaunchKernelGGL((attn_fwd_pl_kernel<T, QK_INT8, CAUSAL, D, SPLIT>), dim3(total), dim3(AT), 0, stream,
                     (const T*)a.q, (const u8*)a.k8, skr, plane, blk, wr, plane, blk,
                     kc ? 1.0f : P_SCALE, (const u8*)a.v8t, a.s, (T*)a.o, a.q_sb, a.q_sh, a.q_sr,
                     a.o_sb, a.o_sh, a.o_sr, (int)a.H, (int)a.H_kv, (int)(a.H / a.H_kv), (int)a.N,
                     (int)a.N_kv, (int)a.N_kv_pad, num_qt, span, a.sm_scale, a.lse, a.kmean,
                     a.vmean);
}

template <typename T, bool QK_INT8, bool CAUSAL>
static void launch_pl_t(const AttnArgs& a, hipStream_t stream) {
  if (a.D == 64)
    launch_pl_d<T, QK_INT8, CAUSAL, 64>(a, stream);
  else
    launch_pl_d<T, QK_INT8, CAUSAL, 128>(a, stream);
}

template <typename T, bool QK_INT8>
static void launch_split_t(const AttnArgs& a, hipStream_t stream) {
  launch_pl_d<T, QK_INT8, false, 64, true>(a, stream);
}

hipError_t launch_attn_fwd_split(const AttnArgs& a, hipStream_t stream) {
  if (a.causal || a.D != 64) return hipErrorInvalidValue;
  if (a.dtype == 1)
    launch_split_t<bf16, false>(a, stream);
  else if (a.qk_int8)
    launch_split_t<f16, true>(a, stream);
  else
    launch_split_t<f16, false>(a, stream);
  return hipGetLastError();
}

hipError_t launch_attn_fwd_pl(const AttnArgs& a, hipStream_t stream) {
  if (a.dtype == 1) {
    if (a.causal)
      launch_pl_t<bf16, false, true>(a, stream);
    else
      launch_pl_t<bf16, false, false>(a, stream);
  } else if (a.qk_int8) {
    if (a.causal)
      launch_pl_t<f16, true, true>(a, stream);
    else
      launch_pl_t<f16, true, false>(a, stream);
  } else {
    if (a.causal)
      launch_pl_t<f16, false, true>(a, stream);
    else
      launch_pl_t<f16, false, false>(a, stream);
  }
  return hipGetLastError();
}

}  // namespace sage
