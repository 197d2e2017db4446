/*
 * sage_mi355.h -- C ABI of the MI355X (gfx950) SageAttention SK1 library, libsagemi355.so.
 *
 * The library quantizes K and V per token (the "prologue") and runs the quantized flash-attention
 * main loop (int8 Q.K on int8 MFMA for fp16 inputs, fp8 Q.K for bf16 inputs, fp8 P.V). It has no
 * torch types: every tensor is a raw device pointer plus int64 element strides, every launch goes on
 * the caller's HIP stream, the library never allocates device memory and never synchronizes the
 * host. Every entry point returns SAGE_OK or a nonzero status; `sage_last_error()` gives the text.
 *
 * Layout vocabulary (the reference's, `sageattention/sk1_backend/sk1_loader.py:405-442`):
 *   Q, K, V, O : logical (B, H, N, D) views, element strides (batch, head, row), last stride 1;
 *                D (head_dim) is 128, or 64 where an entry point takes D
 *   N_pad      : ceil(N/64)*64
 *   K8         : (B*H, N_pad, D) int8 (qk_int8) or fp8 e4m3, row-major
 *   SK, SV     : (B*H, N_pad) fp32 per-token scales
 *   V8T        : (B*H, D, N_pad) fp8 e4m3, V transposed
 *   MEAN       : (B*H, D) fp32 smooth_k mean
 *   S          : (B*H) fp32 per-(b,h) V-scale fold
 * dtype codes: SAGE_F16 = 0, SAGE_BF16 = 1.
 */
#ifndef SAGE_MI355_H
#define SAGE_MI355_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SAGE_OK 0
#define SAGE_ERR_INVALID 1 /* a contract violation: shape, stride, dtype, alignment, size */
#define SAGE_ERR_HIP 2     /* a HIP runtime error (launch, device query) */

#define SAGE_F16 0
#define SAGE_BF16 1

/* main-loop kernel choice of sage_attn_fwd_ex (the first three give the same bits) */
#define SAGE_KERNEL_AUTO 0  /* by grid fill on this device: sage_attn_kernel_choice */
#define SAGE_KERNEL_Q128 1  /* 128 queries per block of 4 waves */
#define SAGE_KERNEL_Q256 2  /* 256 queries per block of 8 waves, two groups in ping-pong */
#define SAGE_KERNEL_PIPE 3  /* 128 queries per block of 4 waves, MFMAs pipelined inside each wave */
#define SAGE_KERNEL_SPLIT 4 /* SAGE_KERNEL_PIPE with the key blocks split between two wave pairs
                               and merged in-block: 64 queries per block; non-causal head_dim 64
                               only (grids that would leave compute units idle); the same P, sums
                               in another order: rounding-level different output bits */

/* Library version as MAJOR*10000 + MINOR*100 + PATCH: 200 (0.2.0). 0.2.0 changed KCONST from
 * three rows per 64-key block to the two above; a caller built against 0.1.0 (100) that allocates
 * or fills KCONST itself must check for 200. */
int sage_version(void);

/* Text of the last error on the calling thread ("" if none). Valid until the next call. */
const char* sage_last_error(void);

/* The build id: a hash of the sources and compiler flags this library was built from (computed by
 * build_lib.py), so that a caller can tell a stale library from one built from its tree. No
 * counterpart in the reference. */
const char* sage_build_id(void);

/*
 * Bytes of device workspace `sage_kv_prologue` (and `sage_kseq_mean`) needs for B*H planes of N
 * rows, for any N_pad. No reference counterpart: the reference allocates its mean with torch per
 * call (`sageattention/sk1_backend/hip_prologue.py:219-222`).
 */
size_t sage_kv_prologue_workspace_bytes(int64_t BH, int64_t N);

/*
 * The smooth_k sequence mean alone: MEAN (B*H, D) fp32 = fp32(sum_n fp64(k[n,d]) / N), the same
 * bits as the `mean` output of sage_kv_prologue (same partial sums, same order). Two launches.
 * Replaces `HipPrologue.kseq_mean` / `h34_kseq_mean_{f16,bf16}`
 * (`sageattention/sk1_backend/hip_prologue.py:267-292`; `kernels/hip/h34_prologue.hip:259-294`).
 *   k          logical (B, H, N, D) view, D = 64 or 128, element strides (k_sb, k_sh, k_sr)
 *   workspace  at least sage_kv_prologue_workspace_bytes(B*H, N) bytes, 256-byte aligned
 */
int sage_kseq_mean(int dtype, const void* k, int64_t k_sb, int64_t k_sh, int64_t k_sr,
                   int64_t B, int64_t H, int64_t N, int64_t D, float* mean, void* workspace,
                   size_t workspace_bytes, void* stream);

/*
 * The K/V prologue: smooth_k mean, per-token K (int8 or fp8) and V (fp8) quantization, and the
 * per-(b,h) V-scale fold, in two launches on `stream`.
 *
 * Replaces `HipPrologue.quant_kv` (`sageattention/sk1_backend/hip_prologue.py:188-244`), its
 * kernels `h34_kseq_mean_{f16,bf16}` (`kernels/hip/h34_prologue.hip:284-294`) and
 * `h34_quant_kv_{f16_i8,f16_f8,bf16_f8}` (`kernels/hip/h34_prologue.hip:214-242`), and
 * `fold_v_scale` (`sageattention/sk1_backend/__init__.py:561-579`).
 *
 *   dtype     SAGE_F16 or SAGE_BF16 (K and V share it)
 *   k_int8    1: K to int8 (fp16 only); 0: K to fp8 e4m3
 *   smooth_k  1: subtract the sequence mean of K first
 *   smooth_v  1: subtract the sequence mean of V (fp64-accumulated, rounded once to fp32, written
 *             to `vmean`) before V's per-token scale and quantization; the main loop adds it back
 *             (sage_attn_fwd_ex's `vmean`). The reference's Triton quantizer's SUB_VMEAN path
 *             (`sageattention/sk1_backend/quant_triton.py:668-678`, `:714-717`) with the
 *             VMEAN epilogue of `kernels/hip/sk1_t6i.hip:290-297`; its shipped HIP prologue
 *             does not produce the mean (`sageattention/sk1_backend/hip_prologue.py:17`).
 *             Costs a third launch (V is read twice).
 *   fold      1: write SV' = SV / S into `sv`; 0: leave SV unfolded (S is written either way)
 *   k, v      logical (B, H, N, D) views with element strides (k_sb, k_sh, k_sr) / (v_...)
 *   D         head_dim, 64 or 128 (64: no counterpart in the reference's shipped path -- its
 *             head_dim-64 object `kernels/hip/sk1_d64.hip` is built but never routed,
 *             `sageattention/sk1_backend/__init__.py:208-229`)
 *   outputs   k8, sk, v8t, sv, s (required); mean (may be NULL; written when smooth_k);
 *             vmean (B*H, 128) fp32 (required with smooth_v, else unused);
 *             kconst (may be NULL): the main loop's per-key constants, (B*H, N_pad/64, 2, 64) fp32:
 *             for each 64-key block SK and RN(SV'*448) -- a layout of SK and SV' that the main
 *             loop stages in one piece per block (no reference counterpart: the reference's
 *             kernel derives them from SK/SV itself, `kernels/hip/sk1_t6i.hip:189-207`, `:249-262`)
 *   workspace at least sage_kv_prologue_workspace_bytes(B*H, N) bytes, 256-byte aligned
 */
int sage_kv_prologue(int dtype, int k_int8, int smooth_k, int smooth_v, int fold,
                     const void* k, int64_t k_sb, int64_t k_sh, int64_t k_sr,
                     const void* v, int64_t v_sb, int64_t v_sh, int64_t v_sr,
                     int64_t B, int64_t H, int64_t N, int64_t N_pad, int64_t D,
                     void* k8, float* sk, void* v8t, float* sv, float* mean, float* vmean,
                     float* s, float* kconst, void* workspace, size_t workspace_bytes,
                     void* stream);

/*
 * `sage_kv_prologue` without the workspace arguments: the prologue's workspace (the fp64 mean
 * partials and per-block V maxima) is a static device array of SAGE_NOALLOC_SCRATCH_BYTES that
 * the library holds on each GPU it runs on until the process ends. No counterpart in the
 * reference: for callers that cannot allocate device memory (code under HIP graph capture, tight
 * serving loops, harnesses that forbid hipMalloc). Nothing is allocated by this call.
 *
 * Limit: a call whose `sage_kv_prologue_workspace_bytes(B*H, N)` exceeds
 * SAGE_NOALLOC_SCRATCH_BYTES returns SAGE_ERR_INVALID ("scratch: ..."); that is every N for
 * B*H <= 768 and B*H up to ~2000 beyond. Every call on one GPU shares that GPU's array: calls that
 * overlap on one GPU (two streams, two host threads) race and must be serialized by the caller.
 * Nothing in the array needs to start at zero (each call writes every partial it reads).
 */
#define SAGE_NOALLOC_SCRATCH_BYTES (4u << 20)
int sage_kv_prologue_noalloc(int dtype, int k_int8, int smooth_k, int smooth_v, int fold,
                             const void* k, int64_t k_sb, int64_t k_sh, int64_t k_sr,
                             const void* v, int64_t v_sb, int64_t v_sh, int64_t v_sr,
                             int64_t B, int64_t H, int64_t N, int64_t N_pad, int64_t D,
                             void* k8, float* sk, void* v8t, float* sv, float* mean, float* vmean,
                             float* s, float* kconst, void* stream);

/*
 * The quantized flash-attention main loop (one launch on `stream`).
 *
 * Replaces `Sk1Attn.launch` / `Sk1Attn.launch_strided`
 * (`sageattention/sk1_backend/sk1_loader.py:628-688`) and their kernels
 * `sk1t6i_attn_fwd_c{0,1}` (`kernels/hip/sk1_t6i.hip:308-316`), `sk1t6in_attn_fwd_c{0,1}`
 * (`kernels/hip/sk1_t6in.hip:323-332`) and `sk1t4a1{sb,nb}_attn_fwd_c{0,1}`
 * (`kernels/hip/sk1_t4a1sb.hip:300-308`). Q is quantized per row inside the kernel (int8 when
 * qk_int8, else fp8 e4m3). The reference's SK and SV' inputs arrive as `kconst`, the prologue's
 * per-key constants (two rows of 64 fp32 per 64-key block: SK, then RN(SV'*448), written from
 * the folded SV'); `s` is the fold S.
 *
 *   q, o   logical (B, H, N, 128) views of `dtype`, element strides (q_sb, q_sh, q_sr) / (o_...)
 *   k8, kconst, v8t, s   the prologue's outputs for the same B, H, N, N_pad and qk_int8
 */
int sage_attn_fwd(int dtype, int qk_int8, int causal,
                  const void* q, int64_t q_sb, int64_t q_sh, int64_t q_sr,
                  const void* k8, const float* kconst, const void* v8t, const float* s,
                  void* o, int64_t o_sb, int64_t o_sh, int64_t o_sr,
                  int64_t B, int64_t H, int64_t N, int64_t N_pad, float sm_scale, void* stream);

/*
 * sage_attn_fwd generalized: grouped K/V heads, a key length of its own, the main-loop kernel
 * chosen by the caller (SAGE_KERNEL_*) and an optional per-row logsumexp. sage_attn_fwd is this
 * with H_kv = H, N_kv = N, SAGE_KERNEL_AUTO and no logsumexp. SAGE_KERNEL_Q128, _Q256 and _PIPE
 * compute the same arithmetic in the same order per query; only the block shape and schedule
 * differ. SAGE_KERNEL_SPLIT runs each query's even and odd 64-key blocks on two waves that
 * exchange their block maxima every block, so each block's probabilities use the sequential
 * running max (the same P as the other kernels), and merges the two row sums and accumulators at
 * the end (each scaled by exp2(mc_i - max(mc0, mc1))): only the fp32 sums round differently. The
 * kernel choice has no counterpart in the reference (one kernel per dtype there).
 *
 *   q, o      logical (B, H, N, D) views, as in sage_attn_fwd
 *   D         head_dim, 64 or 128 (at 64, SAGE_KERNEL_Q256 is refused; at 128 and with causal,
 *             SAGE_KERNEL_SPLIT is refused)
 *   k8, kconst, v8t, s   the prologue's outputs for B*H_kv planes of N_kv keys (N_kv_pad =
 *             ceil(N_kv/64)*64). Query head h reads K/V head h / (H / H_kv) (grouped-query and
 *             multi-query attention; H must be a multiple of H_kv), and N may differ from N_kv
 *             when not causal. The reference's SK1 envelope refuses both
 *             (`sageattention/sk1_backend/__init__.py:966-978`); its upstream API serves them
 *             (`sageattention/core.py:824-829`: H % H_kv == 0, causal only with N == N_kv),
 *             and so does this entry point.
 *
 *   lse    optional (B*H, N) fp32: the natural-log logsumexp of each row's scores times sm_scale,
 *          as `sageattn(..., return_lse=True)` returns it (`core.py:1081-1095`, `:1437-1439` of
 *          the reference): (RN(c_q*m) + log2 l) / 1.44269504 over the quantized scores, plus
 *          sm_scale * (q . kmean) when kmean is given. The reference's SK1 kernels refuse
 *          return_lse (`sageattention/sk1_backend/__init__.py:925-926`); this fills that row.
 *   kmean  optional (B*H_kv, 128) fp32: the smooth_k mean the prologue subtracted (its `mean`
 *          output); used only with lse.
 *   vmean  optional (B*H_kv, 128) fp32: the smooth_v mean the prologue subtracted from V (its
 *          `vmean` output); each output element is then T(fma(acc, S/(l*448), vmean[d])), the
 *          reference's epilogue `acc * inv + vm` (`kernels/hip/sk1_t6i.hip:290-297`). NULL: no
 *          add-back.
 */
int sage_attn_fwd_ex(int dtype, int qk_int8, int causal,
                     const void* q, int64_t q_sb, int64_t q_sh, int64_t q_sr,
                     const void* k8, const float* kconst, const void* v8t, const float* s,
                     void* o, int64_t o_sb, int64_t o_sh, int64_t o_sr,
                     int64_t B, int64_t H, int64_t N, int64_t H_kv, int64_t N_kv,
                     int64_t N_kv_pad, int64_t D, float sm_scale, int kernel,
                     float* lse, const float* kmean, const float* vmean, void* stream);

/*
 * The main-loop kernel SAGE_KERNEL_AUTO runs for a call of this shape: SAGE_KERNEL_Q256,
 * SAGE_KERNEL_PIPE or SAGE_KERNEL_SPLIT (Q128, Q256 and PIPE give the same bits; SPLIT merges two
 * partial row sums and accumulators and differs from them in the last bits of the output). No
 * counterpart in the reference (one kernel per dtype there); for benchmarks and profilers that
 * name the kernel.
 *   cus  compute units to plan for; <= 0: those of the current device (a device query)
 * head_dim 64 runs the key split when not causal and its grid of 64-query blocks,
 * B*H*ceil(N/64), is at most 6 per CU (two rounds: its LDS lets three blocks share a CU), else
 * the pipelined kernel. At 128 the 256-query ping-pong runs when, on `cus` CUs,
 * its grid is estimated to finish at least 3 % sooner: a causal grid with at least 4 of its
 * blocks per CU, unless padding the last query tile to 256 rows costs over 2 % more of the causal
 * work than padding it to 128; a non-causal one by whole rounds of blocks (up to three 128-query
 * blocks or one 256-query block resident per CU) at per-CU throughputs measured on MI355X.
 * Returns the kernel code, or -SAGE_ERR_INVALID for a bad shape or head_dim, or -SAGE_ERR_HIP
 * when the device query fails.
 */
int sage_attn_kernel_choice(int64_t B, int64_t H, int64_t N, int64_t D, int causal, int64_t cus);

/*
 * The main loop on the reference kernel's own inputs: per-key scales SK (B*H_kv, N_kv_pad) and
 * folded value scales SV' (B*H_kv, N_kv_pad) fp32, as the reference's attention kernels take them
 * (`kernels/hip/sk1_t6i.hip:302-306`, `kernels/hip/sk1_t6in.hip:314-320`; the contract of
 * `Sk1Attn._check`, `sageattention/sk1_backend/sk1_loader.py:405-442`), instead of the prologue's
 * KCONST layout. W = RN(SV' * 448) is formed in the kernel with the same single rounding the
 * prologue applies, so for the prologue's SK and SV' the output equals sage_attn_fwd_ex's bit
 * for bit. Runs the software-pipelined kernel (SAGE_KERNEL_PIPE) at every size.
 *   k8, sk, v8t, sv, s   K8, SK, V8T, SV' and S of the scheme for B*H_kv planes of N_kv keys;
 *                        sk and sv 16-byte aligned
 *   vmean                optional (B*H_kv, D) fp32 added to the output (the reference kernel's
 *                        VMEAN, `kernels/hip/sk1_t6i.hip:290-297`)
 *   lse, kmean           as in sage_attn_fwd_ex
 * Other arguments as in sage_attn_fwd_ex.
 */
int sage_attn_fwd_sk(int dtype, int qk_int8, int causal,
                     const void* q, int64_t q_sb, int64_t q_sh, int64_t q_sr,
                     const void* k8, const float* sk, const void* v8t, const float* sv,
                     const float* vmean, const float* s,
                     void* o, int64_t o_sb, int64_t o_sh, int64_t o_sr,
                     int64_t B, int64_t H, int64_t N, int64_t H_kv, int64_t N_kv,
                     int64_t N_kv_pad, int64_t D, float sm_scale,
                     float* lse, const float* kmean, void* stream);

/*
 * Q quantization exactly as the main loop performs it, written out for parity checks.
 * Replaces the in-kernel Q quantization of `kernels/hip/sk1_t6i.hip:91-117` (int8) and
 * `kernels/hip/sk1_t4a1s.hip:79-105` (fp8), which the reference never writes out.
 *   q8  (B*H, N, D) int8 or fp8; sq (B*H, N) fp32 = RN(amax/127) or RN(amax/448);
 *   cq  (B*H, N) fp32 = RN(RN(sm_scale*log2e) * sq)
 */
int sage_quant_q(int dtype, int qk_int8,
                 const void* q, int64_t q_sb, int64_t q_sh, int64_t q_sr,
                 int64_t B, int64_t H, int64_t N, int64_t D, float sm_scale,
                 void* q8, float* sq, float* cq, void* stream);

/*
 * MFMA accumulator layout probe (known-answer test of the fragment layouts the main loop relies
 * on). One wave computes C = A(32x32, int8) * B(32x32, int8) with v_mfma_i32_32x32x32_i8 and
 * D = E(32x64, fp8) * F(64x32, fp8) with v_mfma_scale_f32_32x32x64_f8f6f4, loading operands in
 * the main loop's fragment order and storing results by the assumed accumulator layout.
 * Replaces `kernels/hip/sk1_layout_probe.hip:1-38` (the gfx1201 WMMA probe).
 *   a (32x32 row-major int8, K contiguous), bt (32x32, B transposed: row n holds column n),
 *   c (32x32 int32 out); e (32x64 fp8 row-major), ft (32x64 fp8, F transposed), d (32x32 fp32 out)
 */
int sage_mfma_layout_probe(const void* a, const void* bt, int32_t* c,
                           const void* e, const void* ft, float* d, void* stream);

/*
 * Benchmark probe, not on the served path: the dense rate of the main loop's matrix instructions
 * on this GPU at the clock it runs at (the reference reports its register-resident ceiling beside
 * the documented peak, `docs/METHOD.md:80-91`; no kernel of the reference's library does this).
 * Launches `blocks` blocks of 4 waves; each wave issues `iters` rounds of 4 independent
 * register-resident MFMAs: v_mfma_i32_32x32x32_i8 (qk_int8 != 0) or the e4m3
 * v_mfma_scale_f32_32x32x64_f8f6f4 with unit scales. Ops per launch:
 * blocks * 4 * iters * 4 * 2*32*32*K, K = 32 (int8) or 64 (e4m3). Nothing is read from memory.
 * `clocks` (optional, 2 int64 on the device): the first wave's shader-clock cycles (s_memtime) and
 * constant-rate ticks (s_memrealtime) over its run, i.e. the clock the matrix cores ran at.
 * blocks in [1, 2^20], iters in [1, 2^30].
 */
int sage_mfma_peak_probe(int qk_int8, int64_t blocks, int64_t iters, int64_t* clocks,
                         void* stream);

#ifdef __cplusplus
}
#endif

#endif /* SAGE_MI355_H */
