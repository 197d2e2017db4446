// Host-side launchers shared between the kernel translation units and the C ABI (capi.hip).
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace sage {

// Geometry of the two-launch prologue for BH planes of N rows, padded to N_pad (a multiple of 64,
// at least ceil(N/64)*64). The workspace is sized for head_dim 128, which covers 64.
//   stats pass: C1 blocks per plane (1-D grid of C1*BH), each owning R1 consecutive rows; R1 and
//               C1 follow from Nc = ceil(N/64)*64, and the plane's last block also covers the
//               rows up to N_pad, so extra padding never changes the workspace;
//   quant pass: C2 blocks per plane (1-D grid of C2*BH), each owning R2 rows of N_pad.
// Each grid is one round of resident blocks on MI355X (prologue.hip), so C1 stays small and the
// quant blocks' reduction of the C1 mean partials (128 fp64 each) stays short.
struct PrologueGeom {
  int64_t R1, C1, R2, C2;
};
// cus: the device's compute units; the grids are sized for min(cus, 256) (the workspace bound,
// prologue_workspace_bytes, is the 256-CU geometry's, which has the most mean partials).
PrologueGeom prologue_geom(int64_t BH, int64_t N, int64_t N_pad, int64_t step = 128,
                           int64_t cus = 256);
// bytes of workspace for BH planes of N rows (any N_pad)
size_t prologue_workspace_bytes(int64_t BH, int64_t N);

struct PrologueArgs {
  int dtype, k_int8, smooth_k, smooth_v, fold;
  const void* k;
  int64_t k_sb, k_sh, k_sr;
  const void* v;
  int64_t v_sb, v_sh, v_sr;
  int64_t B, H, N, N_pad;
  int64_t D;       // head_dim: 64 or 128
  void* k8;
  float* sk;
  void* v8t;
  float* sv;
  float* mean;
  float* vmean;    // required with smooth_v: V's sequence mean (B*H, 128) fp32
  float* s;
  float* kconst;   // optional: the main loop's per-key constants (B*H, N_pad/64, 2, 64) fp32
  void* workspace;
  int64_t cus;     // compute units of the launch device (<= 0: 256)
};
hipError_t launch_prologue(const PrologueArgs& a, hipStream_t stream);
// The smooth_k mean alone: K's fp64 column partials (stats pass, K only), then MEAN, with the
// same summation order and rounding as the prologue's MEAN output.
hipError_t launch_kseq_mean(const PrologueArgs& a, hipStream_t stream);

struct AttnArgs {
  int dtype, qk_int8, causal;
  const void* q;
  int64_t q_sb, q_sh, q_sr;
  const void* k8;
  const float* kconst;      // per-key constants in the prologue's KCONST layout, or NULL and:
  const float* sk;          //   SK (B*H_kv, N_kv_pad) and
  const float* svp;         //   SV' (B*H_kv, N_kv_pad), the reference's arrays
  const void* v8t;
  const float* s;
  void* o;
  int64_t o_sb, o_sh, o_sr;
  int64_t B, H, N;          // query side: B*H planes of N rows
  int64_t D;                // head_dim: 64 or 128 (the 256-query kernel serves 128 only)
  int64_t H_kv, N_kv, N_kv_pad;   // key/value side: B*H_kv planes of N_kv rows (H % H_kv == 0)
  float sm_scale;
  float* lse;              // optional (B*H, N) fp32 row logsumexp
  const float* kmean;      // optional (B*H_kv, 128) fp32 smooth_k mean, for the logsumexp correction
  const float* vmean;      // optional (B*H_kv, 128) fp32 smooth_v mean, added to the output
};
hipError_t launch_attn_fwd(const AttnArgs& a, hipStream_t stream);
// the two-group ping-pong form of the same main loop (256 queries per block of 8 waves)
hipError_t launch_attn_fwd_pp(const AttnArgs& a, hipStream_t stream);
// the software-pipelined form (128 queries per block of 4 waves, three or four blocks per CU)
hipError_t launch_attn_fwd_pl(const AttnArgs& a, hipStream_t stream);
// the same kernel in its key-split form (non-causal, head_dim 64; 64 queries per block, the even
// and the odd key blocks run by two wave pairs that exchange their block maxima, merged in LDS)
hipError_t launch_attn_fwd_split(const AttnArgs& a, hipStream_t stream);

struct QuantQArgs {
  int dtype, qk_int8;
  const void* q;
  int64_t q_sb, q_sh, q_sr;
  int64_t B, H, N;
  int64_t D;       // head_dim: 64 or 128
  float sm_scale;
  void* q8;
  float* sq;
  float* cq;
};
hipError_t launch_quant_q(const QuantQArgs& a, hipStream_t stream);

hipError_t launch_layout_probe(const void* a, const void* bt, int32_t* c, const void* e,
                               const void* ft, float* d, hipStream_t stream);
// MFMA throughput probe: blocks x 256 threads, each wave `iters` rounds of 4 independent MFMAs.
hipError_t launch_mfma_peak(bool int8, int64_t blocks, int64_t iters, int64_t* clocks,
                            hipStream_t stream);

}  // namespace sage
