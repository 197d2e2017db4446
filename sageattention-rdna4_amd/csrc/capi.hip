// The C ABI of libsagemi355.so (declared in include/sage_mi355.h): argument contracts, error
// reporting, and the calls into the kernel launchers. Nothing here allocates device memory or
// synchronizes the host.
#include <stdarg.h>
#include <stdio.h>

#include <atomic>
#include <mutex>
#include <string>

#include "../../include/sage_mi355.h"
#include "sage_launch.h"

namespace {

thread_local std::string g_err;

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_err = buf;
  return code;
}

int hip_status(hipError_t e, const char* what) {
  if (e == hipSuccess) {
    g_err.clear();
    return SAGE_OK;
  }
  return fail(SAGE_ERR_HIP, "%s: %s (%s)", what, hipGetErrorName(e), hipGetErrorString(e));
}

constexpr int64_t kInt32Max = 2147483647LL;

bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

// The stride rule of the 16-byte vector accesses (the reference's `strided_view_reason`,
// sageattention/sk1_backend/sk1_loader.py:313-369): positive, multiples of 8 elements.
int check_view(const char* name, const void* p, int64_t sb, int64_t sh, int64_t sr) {
  if (p == nullptr) return fail(SAGE_ERR_INVALID, "%s is NULL", name);
  if (!aligned16(p)) return fail(SAGE_ERR_INVALID, "%s: ptr_align (pointer not 16-byte aligned)", name);
  if (sb <= 0 || sh <= 0 || sr <= 0)
    return fail(SAGE_ERR_INVALID, "%s: stride_nonpos (%lld, %lld, %lld)", name, (long long)sb,
                (long long)sh, (long long)sr);
  if ((sb | sh | sr) & 7)
    return fail(SAGE_ERR_INVALID, "%s: stride_align (strides must be multiples of 8 elements)", name);
  return SAGE_OK;
}

int check_shape(int64_t B, int64_t H, int64_t N, int64_t N_pad) {
  if (B < 1 || H < 1) return fail(SAGE_ERR_INVALID, "B and H must be >= 1 (B=%lld H=%lld)",
                                  (long long)B, (long long)H);
  if (N < 1) return fail(SAGE_ERR_INVALID, "n_lt_1: N must be >= 1 (N=%lld)", (long long)N);
  if (N_pad < N || (N_pad % 64) != 0)
    return fail(SAGE_ERR_INVALID, "n_pad: N_pad must be a multiple of 64 and >= N (N=%lld N_pad=%lld)",
                (long long)N, (long long)N_pad);
  // A plane's padded rows must fit the 32-bit in-plane offsets of the main loop's staging; the
  // grids themselves are bounded per launch (check_grid).
  if (N_pad > kInt32Max / 128 || B > kInt32Max || H > kInt32Max || B * H > kInt32Max)
    return fail(SAGE_ERR_INVALID, "grid: shape too large (B*H=%lld N=%lld)", (long long)(B * H),
                (long long)N);
  return SAGE_OK;
}

// Every grid is a 1-D list of blocks, so B*H has no limit of its own; HIP bounds one launch at
// 2^32 - 1 threads (blocks times threads per block).
int check_grid(const char* what, int64_t blocks, int64_t threads) {
  if (blocks < 1 || blocks > (int64_t)(0xFFFFFFFFull / (uint64_t)threads))
    return fail(SAGE_ERR_INVALID,
                "grid: %s needs %lld blocks of %lld threads, beyond HIP's 2^32-1 threads per launch",
                what, (long long)blocks, (long long)threads);
  return SAGE_OK;
}

// The main-loop grids: 128-query blocks of 256 threads (SAGE_KERNEL_Q128, SAGE_KERNEL_PIPE) and
// 256-query blocks of 512 threads (SAGE_KERNEL_Q256). Checked for every kernel, so the refusal
// does not depend on the automatic choice. The key split's 64-query grid (SAGE_KERNEL_SPLIT) is
// checked when that kernel is asked for; the automatic choice takes it only for grids of at most
// six of its blocks per compute unit.
int check_main_grid(int64_t B, int64_t H, int64_t N) {
  int rc = check_grid("the 128-query main loop", B * H * ((N + 127) / 128), 256);
  if (rc) return rc;
  return check_grid("the 256-query main loop", B * H * ((N + 255) / 256), 512);
}

// The prologue's two passes: C1 and C2 blocks per plane of 256 threads.
int check_prologue_grid(int64_t BH, int64_t N, int64_t N_pad) {
  const sage::PrologueGeom g = sage::prologue_geom(BH, N, N_pad);
  const int64_t c = g.C1 > g.C2 ? g.C1 : g.C2;
  if (c > kInt32Max / BH) return check_grid("the prologue", kInt32Max, 256);
  return check_grid("the prologue", c * BH, 256);
}

int check_head_dim(int64_t D) {
  if (D != 64 && D != 128)
    return fail(SAGE_ERR_INVALID, "head_dim: D must be 64 or 128 (got %lld)", (long long)D);
  return SAGE_OK;
}

}  // namespace

// The workspace of sage_kv_prologue_noalloc: one copy per GPU, loaded with the code object and held
// until the process ends. Host code never passes `scratch` itself (on the host it names a
// stand-in, not device memory): it passes the device address that hipGetSymbolAddress returns for
// the current device, kept in g_scratch_ptr.
static __device__ __align__(256) unsigned char scratch[SAGE_NOALLOC_SCRATCH_BYTES];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// The current device's address of `scratch`, looked up once per device with that device current.
int scratch_for_current_device(void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_status(e, "sage_kv_prologue_noalloc hipGetDevice");
  if (dev < 0 || dev >= kMaxDevices)
    return fail(SAGE_ERR_INVALID, "scratch: device %d beyond the %d the library tracks", dev,
                kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return hip_status(e, "sage_kv_prologue_noalloc hipGetSymbolAddress");
    if (p == nullptr || ((uintptr_t)p & 255u))
      return fail(SAGE_ERR_HIP, "scratch: hipGetSymbolAddress gave an unusable address %p", p);
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return SAGE_OK;
}

// Compute units of the current device, looked up once per device.
std::atomic<int> g_cus[kMaxDevices];

int cus_of_current_device(int64_t* out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_status(e, "hipGetDevice");
  if (dev < 0 || dev >= kMaxDevices)
    return fail(SAGE_ERR_INVALID, "device %d beyond the %d the library tracks", dev, kMaxDevices);
  int n = g_cus[dev].load(std::memory_order_relaxed);
  if (n <= 0) {
    e = hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev);
    if (e != hipSuccess) return hip_status(e, "hipDeviceGetAttribute(multiprocessor count)");
    if (n <= 0) return fail(SAGE_ERR_HIP, "device %d reports %d compute units", dev, n);
    g_cus[dev].store(n, std::memory_order_relaxed);
  }
  *out = n;
  return SAGE_OK;
}

// Estimated makespans of a non-causal grid, in units of one 128-query block's work run alone on a
// CU. Every block of a non-causal grid does the same work, and the dispatcher keeps each CU's
// slots full, so the grid runs in rounds. Per-CU throughputs, measured on MI355X (B*H = 8 and 48,
// N = 288 .. 32768, both kernels timed on one box): the 128-query kernels with 1, 2 or 3 blocks
// resident on a CU (one to three waves per SIMD) 1.00, 1.52 and 1.69; the 256-query ping-pong
// (one block per CU) 1.75 blocks of 128 queries.
double est_q128(int64_t blocks, int64_t cus) {
  static const double rate[4] = {0.0, 1.0, 1.52, 1.69};
  const int64_t full = blocks / (3 * cus), rem = blocks - full * 3 * cus;
  double t = (double)full * 3.0 / rate[3];
  if (rem) {
    const int64_t k = (rem + cus - 1) / cus;
    t += (double)k / rate[k];
  }
  return t;
}
double est_q256(int64_t blocks, int64_t cus) {
  return (double)((blocks + cus - 1) / cus) * 2.0 / 1.75;
}

// Causal: the padded rows of a plane's last query tile are its longest rows, so padding to
// `tile` rows adds about 2 * pad / N of the plane's causal work.
double causal_pad_work(int64_t N, int64_t tile) {
  return 2.0 * (double)((N + tile - 1) / tile * tile - N) / (double)N;
}

int kernel_for(int64_t B, int64_t H, int64_t N, int64_t D, int causal, int64_t cus) {
  if (D != 128) {
    // head_dim 64, non-causal, with at most six of the key split's 64-query blocks per CU (two
    // rounds of three, its LDS bound): twice the waves, each over half the keys. Measured on
    // MI355X, 1.01-1.57x faster than the pipelined kernel there (1.24x at SDXL's 2.5 per CU);
    // from about 8 per CU on the pipelined kernel's four resident blocks per CU catch up and
    // from 12 on they win (0.95x at 16 and 32 per CU).
    const int64_t nb64 = B * H * ((N + 63) / 64);
    return (!causal && nb64 <= 6 * cus) ? SAGE_KERNEL_SPLIT : SAGE_KERNEL_PIPE;
  }
  const int64_t nb256 = B * H * ((N + 255) / 256);
  if (causal)
    return (nb256 >= 4 * cus && causal_pad_work(N, 256) - causal_pad_work(N, 128) < 0.02)
               ? SAGE_KERNEL_Q256
               : SAGE_KERNEL_PIPE;
  const int64_t nb128 = B * H * ((N + 127) / 128);
  return est_q256(nb256, cus) < 0.97 * est_q128(nb128, cus) ? SAGE_KERNEL_Q256
                                                              : SAGE_KERNEL_PIPE;
}

}  // namespace

extern "C" {

int sage_attn_kernel_choice(int64_t B, int64_t H, int64_t N, int64_t D, int causal, int64_t cus) {
  if (B < 1 || H < 1 || N < 1)
    return -fail(SAGE_ERR_INVALID, "shape: B, H and N must be positive (B=%lld H=%lld N=%lld)",
                 (long long)B, (long long)H, (long long)N);
  if (D != 64 && D != 128)
    return -fail(SAGE_ERR_INVALID, "head_dim: %lld is not 64 or 128", (long long)D);
  if (cus <= 0) {
    const int rc = cus_of_current_device(&cus);
    if (rc) return -rc;
  }
  return kernel_for(B, H, N, D, causal, cus);
}

int sage_version(void) { return 200; }

#ifndef SAGE_BUILD_ID
#define SAGE_BUILD_ID "unknown"
#endif
const char* sage_build_id(void) { return SAGE_BUILD_ID; }

const char* sage_last_error(void) { return g_err.c_str(); }

size_t sage_kv_prologue_workspace_bytes(int64_t BH, int64_t N) {
  if (BH < 1 || N < 1) return 0;
  return sage::prologue_workspace_bytes(BH, N);
}

int sage_kv_prologue(int dtype, int k_int8, int smooth_k, int smooth_v, int fold, const void* k,
                     int64_t k_sb, int64_t k_sh, int64_t k_sr, const void* v, int64_t v_sb,
                     int64_t v_sh, int64_t v_sr, int64_t B, int64_t H, int64_t N, int64_t N_pad,
                     int64_t D, void* k8, float* sk, void* v8t, float* sv, float* mean,
                     float* vmean,
                     float* s, float* kconst, void* workspace, size_t workspace_bytes,
                     void* stream) {
  if (dtype != SAGE_F16 && dtype != SAGE_BF16)
    return fail(SAGE_ERR_INVALID, "dtype: unsupported dtype code %d", dtype);
  if (dtype == SAGE_BF16 && k_int8)
    return fail(SAGE_ERR_INVALID, "bf16_int8: int8 K is served for fp16 inputs only");
  int rc = check_shape(B, H, N, N_pad);
  if (rc) return rc;
  if ((rc = check_prologue_grid(B * H, N, N_pad))) return rc;
  if ((rc = check_head_dim(D))) return rc;
  if ((rc = check_view("k", k, k_sb, k_sh, k_sr))) return rc;
  if ((rc = check_view("v", v, v_sb, v_sh, v_sr))) return rc;
  if (!k8 || !sk || !v8t || !sv || !s) return fail(SAGE_ERR_INVALID, "an output pointer is NULL");
  if (smooth_v && !vmean)
    return fail(SAGE_ERR_INVALID, "vmean: smooth_v needs the vmean output (B*H x 128 fp32)");
  if (!aligned16(k8) || !aligned16(v8t) || !aligned16(sk) || !aligned16(sv) || !aligned16(kconst))
    return fail(SAGE_ERR_INVALID, "ptr_align: outputs must be 16-byte aligned");
  const size_t need = sage::prologue_workspace_bytes(B * H, N);
  if (workspace == nullptr || workspace_bytes < need || ((uintptr_t)workspace & 255u))
    return fail(SAGE_ERR_INVALID, "workspace: need %zu bytes, 256-byte aligned (got %zu)", need,
                workspace_bytes);
  int64_t cus = 0;
  if ((rc = cus_of_current_device(&cus))) return rc;
  sage::PrologueArgs a;
  a.cus = cus;
  a.dtype = dtype;
  a.k_int8 = k_int8 ? 1 : 0;
  a.smooth_k = smooth_k ? 1 : 0;
  a.smooth_v = smooth_v ? 1 : 0;
  a.fold = fold ? 1 : 0;
  a.k = k;
  a.k_sb = k_sb;
  a.k_sh = k_sh;
  a.k_sr = k_sr;
  a.v = v;
  a.v_sb = v_sb;
  a.v_sh = v_sh;
  a.v_sr = v_sr;
  a.B = B;
  a.H = H;
  a.N = N;
  a.N_pad = N_pad;
  a.D = D;
  a.k8 = k8;
  a.sk = sk;
  a.v8t = v8t;
  a.sv = sv;
  a.mean = smooth_k ? mean : nullptr;
  a.vmean = smooth_v ? vmean : nullptr;
  a.s = s;
  a.kconst = kconst;
  a.workspace = workspace;
  return hip_status(sage::launch_prologue(a, (hipStream_t)stream), "sage_kv_prologue launch");
}

int sage_kv_prologue_noalloc(int dtype, int k_int8, int smooth_k, int smooth_v, int fold,
                             const void* k, int64_t k_sb, int64_t k_sh, int64_t k_sr,
                             const void* v, int64_t v_sb, int64_t v_sh, int64_t v_sr, int64_t B,
                             int64_t H, int64_t N, int64_t N_pad, int64_t D, void* k8, float* sk,
                             void* v8t, float* sv, float* mean, float* vmean, float* s,
                             float* kconst, void* stream) {
  int rc = check_shape(B, H, N, N_pad);
  if (rc) return rc;
  const size_t need = sage::prologue_workspace_bytes(B * H, N);
  if (need > (size_t)SAGE_NOALLOC_SCRATCH_BYTES)
    return fail(SAGE_ERR_INVALID,
                "scratch: B*H=%lld N=%lld needs a %zu-byte workspace, the static scratch holds %zu "
                "(use sage_kv_prologue with a workspace of that size)",
                (long long)(B * H), (long long)N, need, (size_t)SAGE_NOALLOC_SCRATCH_BYTES);
  void* ws = nullptr;
  if ((rc = scratch_for_current_device(&ws))) return rc;
  return sage_kv_prologue(dtype, k_int8, smooth_k, smooth_v, fold, k, k_sb, k_sh, k_sr, v, v_sb,
                          v_sh, v_sr, B, H, N, N_pad, D, k8, sk, v8t, sv, mean, vmean, s, kconst,
                          ws, (size_t)SAGE_NOALLOC_SCRATCH_BYTES, stream);
}

int sage_attn_fwd_ex(int dtype, int qk_int8, int causal, const void* q, int64_t q_sb,
                     int64_t q_sh, int64_t q_sr, const void* k8, const float* kconst,
                     const void* v8t, const float* s, void* o, int64_t o_sb, int64_t o_sh,
                     int64_t o_sr, int64_t B, int64_t H, int64_t N, int64_t H_kv, int64_t N_kv,
                     int64_t N_kv_pad, int64_t D, float sm_scale, int kernel, float* lse,
                     const float* kmean, const float* vmean, void* stream) {
  if (dtype != SAGE_F16 && dtype != SAGE_BF16)
    return fail(SAGE_ERR_INVALID, "dtype: unsupported dtype code %d", dtype);
  if (dtype == SAGE_BF16 && qk_int8)
    return fail(SAGE_ERR_INVALID, "bf16_int8: int8 Q.K is served for fp16 inputs only");
  int rc = check_shape(B, H, N, (N + 63) / 64 * 64);
  if (rc) return rc;
  if ((rc = check_main_grid(B, H, N))) return rc;
  if (H_kv < 1 || H % H_kv != 0)
    return fail(SAGE_ERR_INVALID, "heads: H (%lld) must be a multiple of H_kv (%lld)",
                (long long)H, (long long)H_kv);
  if ((rc = check_shape(B, H_kv, N_kv, N_kv_pad))) return rc;
  if (causal && N != N_kv)
    return fail(SAGE_ERR_INVALID, "seq_len: causal attention needs N == N_kv (N=%lld N_kv=%lld)",
                (long long)N, (long long)N_kv);
  if ((rc = check_head_dim(D))) return rc;
  if (D == 64 && kernel == SAGE_KERNEL_Q256)
    return fail(SAGE_ERR_INVALID, "kernel: the 256-query kernel serves head_dim 128 only");
  if (kernel == SAGE_KERNEL_SPLIT && (causal || D != 64))
    return fail(SAGE_ERR_INVALID,
                "kernel: the key-split kernel serves non-causal head_dim 64 calls only");
  if ((rc = check_view("q", q, q_sb, q_sh, q_sr))) return rc;
  if ((rc = check_view("o", o, o_sb, o_sh, o_sr))) return rc;
  if (!k8 || !kconst || !v8t || !s) return fail(SAGE_ERR_INVALID, "an input pointer is NULL");
  if (!aligned16(k8) || !aligned16(v8t) || !aligned16(kconst))
    return fail(SAGE_ERR_INVALID, "ptr_align: quantized inputs must be 16-byte aligned");
  if (!(sm_scale > 0.0f) || !(sm_scale < 3.0e38f))
    return fail(SAGE_ERR_INVALID, "sm_scale: must be positive and finite (got %g)", (double)sm_scale);
  if (kernel != SAGE_KERNEL_AUTO && kernel != SAGE_KERNEL_Q128 && kernel != SAGE_KERNEL_Q256 &&
      kernel != SAGE_KERNEL_PIPE && kernel != SAGE_KERNEL_SPLIT)
    return fail(SAGE_ERR_INVALID, "kernel: unknown main-loop kernel code %d", kernel);
  if (lse && ((uintptr_t)lse & 3u))
    return fail(SAGE_ERR_INVALID, "ptr_align: lse must be 4-byte aligned");
  if (kmean && !aligned16(kmean))
    return fail(SAGE_ERR_INVALID, "ptr_align: kmean must be 16-byte aligned");
  if (vmean && !aligned16(vmean))
    return fail(SAGE_ERR_INVALID, "ptr_align: vmean must be 16-byte aligned");
  sage::AttnArgs a;
  a.dtype = dtype;
  a.qk_int8 = qk_int8 ? 1 : 0;
  a.causal = causal ? 1 : 0;
  a.q = q;
  a.q_sb = q_sb;
  a.q_sh = q_sh;
  a.q_sr = q_sr;
  a.k8 = k8;
  a.kconst = kconst;
  a.sk = nullptr;
  a.svp = nullptr;
  a.v8t = v8t;
  a.s = s;
  a.o = o;
  a.o_sb = o_sb;
  a.o_sh = o_sh;
  a.o_sr = o_sr;
  a.B = B;
  a.H = H;
  a.N = N;
  a.H_kv = H_kv;
  a.N_kv = N_kv;
  a.N_kv_pad = N_kv_pad;
  a.D = D;
  a.sm_scale = sm_scale;
  a.lse = lse;
  a.kmean = lse ? kmean : nullptr;
  a.vmean = vmean;
  // SAGE_KERNEL_AUTO: the kernel the grid-fill rule picks for this device (kernel_for)
  if (kernel == SAGE_KERNEL_AUTO) {
    int64_t cus = 0;
    if ((rc = cus_of_current_device(&cus))) return rc;
    kernel = kernel_for(B, H, N, D, causal, cus);
  }
  if (kernel == SAGE_KERNEL_SPLIT &&
      (rc = check_grid("the key-split main loop", B * H * ((N + 63) / 64), 256)))
    return rc;
  hipError_t e;
  if (kernel == SAGE_KERNEL_PIPE)
    e = sage::launch_attn_fwd_pl(a, (hipStream_t)stream);
  else if (kernel == SAGE_KERNEL_SPLIT)
    e = sage::launch_attn_fwd_split(a, (hipStream_t)stream);
  else if (kernel == SAGE_KERNEL_Q256)
    e = sage::launch_attn_fwd_pp(a, (hipStream_t)stream);
  else
    e = sage::launch_attn_fwd(a, (hipStream_t)stream);
  return hip_status(e, "sage_attn_fwd launch");
}

int sage_attn_fwd_sk(int dtype, int qk_int8, int causal, const void* q, int64_t q_sb,
                     int64_t q_sh, int64_t q_sr, const void* k8, const float* sk,
                     const void* v8t, const float* sv, const float* vmean, const float* s,
                     void* o, int64_t o_sb, int64_t o_sh, int64_t o_sr, int64_t B, int64_t H,
                     int64_t N, int64_t H_kv, int64_t N_kv, int64_t N_kv_pad, int64_t D,
                     float sm_scale, float* lse, const float* kmean, void* stream) {
  if (dtype != SAGE_F16 && dtype != SAGE_BF16)
    return fail(SAGE_ERR_INVALID, "dtype: unsupported dtype code %d", dtype);
  if (dtype == SAGE_BF16 && qk_int8)
    return fail(SAGE_ERR_INVALID, "bf16_int8: int8 Q.K is served for fp16 inputs only");
  int rc = check_shape(B, H, N, (N + 63) / 64 * 64);
  if (rc) return rc;
  if ((rc = check_main_grid(B, H, N))) return rc;
  if (H_kv < 1 || H % H_kv != 0)
    return fail(SAGE_ERR_INVALID, "heads: H (%lld) must be a multiple of H_kv (%lld)",
                (long long)H, (long long)H_kv);
  if ((rc = check_shape(B, H_kv, N_kv, N_kv_pad))) return rc;
  if (causal && N != N_kv)
    return fail(SAGE_ERR_INVALID, "seq_len: causal attention needs N == N_kv (N=%lld N_kv=%lld)",
                (long long)N, (long long)N_kv);
  if ((rc = check_head_dim(D))) return rc;
  if ((rc = check_view("q", q, q_sb, q_sh, q_sr))) return rc;
  if ((rc = check_view("o", o, o_sb, o_sh, o_sr))) return rc;
  if (!k8 || !sk || !v8t || !sv || !s) return fail(SAGE_ERR_INVALID, "an input pointer is NULL");
  // the per-key rows are staged 256 bytes per 64-key block
  if (!aligned16(k8) || !aligned16(v8t) || !aligned16(sk) || !aligned16(sv))
    return fail(SAGE_ERR_INVALID, "ptr_align: quantized inputs and scales must be 16-byte aligned");
  if (!(sm_scale > 0.0f) || !(sm_scale < 3.0e38f))
    return fail(SAGE_ERR_INVALID, "sm_scale: must be positive and finite (got %g)", (double)sm_scale);
  if (lse && ((uintptr_t)lse & 3u))
    return fail(SAGE_ERR_INVALID, "ptr_align: lse must be 4-byte aligned");
  if (kmean && !aligned16(kmean))
    return fail(SAGE_ERR_INVALID, "ptr_align: kmean must be 16-byte aligned");
  if (vmean && !aligned16(vmean))
    return fail(SAGE_ERR_INVALID, "ptr_align: vmean must be 16-byte aligned");
  sage::AttnArgs a;
  a.dtype = dtype;
  a.qk_int8 = qk_int8 ? 1 : 0;
  a.causal = causal ? 1 : 0;
  a.q = q;
  a.q_sb = q_sb;
  a.q_sh = q_sh;
  a.q_sr = q_sr;
  a.k8 = k8;
  a.kconst = nullptr;
  a.sk = sk;
  a.svp = sv;
  a.v8t = v8t;
  a.s = s;
  a.o = o;
  a.o_sb = o_sb;
  a.o_sh = o_sh;
  a.o_sr = o_sr;
  a.B = B;
  a.H = H;
  a.N = N;
  a.H_kv = H_kv;
  a.N_kv = N_kv;
  a.N_kv_pad = N_kv_pad;
  a.D = D;
  a.sm_scale = sm_scale;
  a.lse = lse;
  a.kmean = lse ? kmean : nullptr;
  a.vmean = vmean;
  return hip_status(sage::launch_attn_fwd_pl(a, (hipStream_t)stream), "sage_attn_fwd_sk launch");
}

int sage_kseq_mean(int dtype, const void* k, int64_t k_sb, int64_t k_sh, int64_t k_sr,
                   int64_t B, int64_t H, int64_t N, int64_t D, float* mean, void* workspace,
                   size_t workspace_bytes, void* stream) {
  if (dtype != SAGE_F16 && dtype != SAGE_BF16)
    return fail(SAGE_ERR_INVALID, "mean_dtype: unsupported dtype code %d", dtype);
  const int64_t N_pad = (N + 63) / 64 * 64;
  int rc = check_shape(B, H, N, N_pad);
  if (rc) return rc;
  if ((rc = check_prologue_grid(B * H, N, N_pad))) return rc;
  if (D != 64 && D != 128)
    return fail(SAGE_ERR_INVALID, "mean_head_dim: D must be 64 or 128 (got %lld)", (long long)D);
  if ((rc = check_view("k", k, k_sb, k_sh, k_sr))) return rc;
  if (!mean) return fail(SAGE_ERR_INVALID, "an output pointer is NULL");
  const size_t need = sage::prologue_workspace_bytes(B * H, N);
  if (workspace == nullptr || workspace_bytes < need || ((uintptr_t)workspace & 255u))
    return fail(SAGE_ERR_INVALID, "workspace: need %zu bytes, 256-byte aligned (got %zu)", need,
                workspace_bytes);
  int64_t cus = 0;
  if ((rc = cus_of_current_device(&cus))) return rc;
  sage::PrologueArgs a = {};
  a.cus = cus;
  a.dtype = dtype;
  a.smooth_k = 1;
  a.k = k;
  a.k_sb = k_sb;
  a.k_sh = k_sh;
  a.k_sr = k_sr;
  a.B = B;
  a.H = H;
  a.N = N;
  a.N_pad = N_pad;
  a.D = D;
  a.mean = mean;
  a.workspace = workspace;
  return hip_status(sage::launch_kseq_mean(a, (hipStream_t)stream), "sage_kseq_mean launch");
}

int sage_attn_fwd(int dtype, int qk_int8, int causal, const void* q, int64_t q_sb, int64_t q_sh,
                  int64_t q_sr, const void* k8, const float* kconst, const void* v8t,
                  const float* s, void* o, int64_t o_sb, int64_t o_sh, int64_t o_sr, int64_t B,
                  int64_t H, int64_t N, int64_t N_pad, float sm_scale, void* stream) {
  return sage_attn_fwd_ex(dtype, qk_int8, causal, q, q_sb, q_sh, q_sr, k8, kconst, v8t, s, o,
                          o_sb, o_sh, o_sr, B, H, N, H, N, N_pad, 128, sm_scale,
                          SAGE_KERNEL_AUTO, nullptr, nullptr, nullptr, stream);
}

int sage_quant_q(int dtype, int qk_int8, const void* q, int64_t q_sb, int64_t q_sh, int64_t q_sr,
                 int64_t B, int64_t H, int64_t N, int64_t D, float sm_scale, void* q8, float* sq,
                 float* cq, void* stream) {
  if (dtype != SAGE_F16 && dtype != SAGE_BF16)
    return fail(SAGE_ERR_INVALID, "dtype: unsupported dtype code %d", dtype);
  if (dtype == SAGE_BF16 && qk_int8)
    return fail(SAGE_ERR_INVALID, "bf16_int8: int8 Q is served for fp16 inputs only");
  int rc = check_shape(B, H, N, (N + 63) / 64 * 64);
  if (rc) return rc;
  if ((rc = check_grid("the Q quantizer", B * H * ((N + 31) / 32), 64))) return rc;
  if ((rc = check_head_dim(D))) return rc;
  if ((rc = check_view("q", q, q_sb, q_sh, q_sr))) return rc;
  if (!q8 || !sq || !cq) return fail(SAGE_ERR_INVALID, "an output pointer is NULL");
  if (!aligned16(q8)) return fail(SAGE_ERR_INVALID, "ptr_align: q8 must be 16-byte aligned");
  sage::QuantQArgs a;
  a.dtype = dtype;
  a.qk_int8 = qk_int8 ? 1 : 0;
  a.q = q;
  a.q_sb = q_sb;
  a.q_sh = q_sh;
  a.q_sr = q_sr;
  a.B = B;
  a.H = H;
  a.N = N;
  a.D = D;
  a.sm_scale = sm_scale;
  a.q8 = q8;
  a.sq = sq;
  a.cq = cq;
  return hip_status(sage::launch_quant_q(a, (hipStream_t)stream), "sage_quant_q launch");
}

int sage_mfma_layout_probe(const void* a, const void* bt, int32_t* c, const void* e,
                           const void* ft, float* d, void* stream) {
  if (!a || !bt || !c || !e || !ft || !d) return fail(SAGE_ERR_INVALID, "a pointer is NULL");
  if (!aligned16(a) || !aligned16(bt) || !aligned16(e) || !aligned16(ft))
    return fail(SAGE_ERR_INVALID, "ptr_align: operands must be 16-byte aligned");
  return hip_status(sage::launch_layout_probe(a, bt, c, e, ft, d, (hipStream_t)stream),
                    "sage_mfma_layout_probe launch");
}

int sage_mfma_peak_probe(int qk_int8, int64_t blocks, int64_t iters, int64_t* clocks,
                         void* stream) {
  if (blocks < 1 || blocks > (1 << 20))
    return fail(SAGE_ERR_INVALID, "blocks must be in [1, 2^20] (got %lld)", (long long)blocks);
  if (iters < 1 || iters > (1LL << 30))
    return fail(SAGE_ERR_INVALID, "iters must be in [1, 2^30] (got %lld)", (long long)iters);
  if (clocks != nullptr && ((uintptr_t)clocks & 7u))
    return fail(SAGE_ERR_INVALID, "clocks must be 8-byte aligned");
  return hip_status(sage::launch_mfma_peak(qk_int8 != 0, blocks, iters, clocks, (hipStream_t)stream),
                    "sage_mfma_peak_probe launch");
}

}  // extern "C"
