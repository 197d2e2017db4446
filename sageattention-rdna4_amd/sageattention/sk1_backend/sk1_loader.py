"""ctypes binding of libsagemi355.so and the tensor contract of its launches.

The reference binds prebuilt code objects through `hipModuleLoadData` on torch's HIP runtime
(`sageattention/sk1_backend/sk1_loader.py:129-299` of the reference). This build instead loads one
C-ABI shared library (`include/sage_mi355.h`) compiled for gfx950. `torch` is imported first, so the
library's `libamdhip64.so.7` dependency resolves to the HIP runtime torch already loaded: one runtime
image per process, and torch's stream handles are valid in the library.

Every launch goes on `torch.cuda.current_stream()` with no host synchronization
(`sk1_loader.py:17-19`, `:301-303` of the reference).
"""
import ctypes
import os
import threading

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.environ.get(
    "SAGE_MI355_LIB", os.path.join(os.path.dirname(_HERE), "_lib", "libsagemi355.so"))

SAGE_F16, SAGE_BF16 = 0, 1

#: Every reason `strided_view_reason` can return, in evaluation order. The strings are the
#: reference's refusal vocabulary (`sageattention/sk1_backend/sk1_loader.py:308-309`); its
#: `stride_int32` is not among them (see below).
STRIDED_REFUSALS = ("rank", "stride_last", "stride_nonpos", "stride_align", "ptr_align",
                    "stride_overlap")


def strided_view_reason(t, name="t"):
    """`None` if `t` is a servable logical (B, H, N, D) view, else the refusal reason.

    Derived from this build's kernels, which read Q/K/V and write O with 16-byte vector accesses
    through int64 (batch, head, row) strides: rank 4; last stride 1 (the 16-byte accesses run
    along D); every stride positive and the outer three multiples of 8 elements (each access
    16-byte aligned); a 16-byte-aligned pointer; an injective index map, so that no two output
    rows alias (sizes-1 dims dropped, strides sorted, each at least the previous stride times its
    size). The reference's rule (`sageattention/sk1_backend/sk1_loader.py:313-369`) also refuses
    strides beyond int32 (`stride_int32`), because its kernels take int strides; every address
    here is formed in 64 bits, so no such refusal is needed.
    """
    if t.dim() != 4:
        return "rank"
    st = t.stride()
    if t.is_contiguous() and st[3] == 1 and st[0] > 0 and st[1] > 0 and st[2] > 0 \
            and not ((st[0] | st[1] | st[2]) & 7) and not (t.data_ptr() & 15):
        return None   # row-major with positive strides: an injective index map
    if int(t.stride(3)) != 1:
        return "stride_last"
    st = [int(s) for s in st]
    if any(s <= 0 for s in st):
        return "stride_nonpos"
    if any(st[i] % 8 for i in (0, 1, 2)):
        return "stride_align"
    if int(t.data_ptr()) % 16:
        return "ptr_align"
    dims = sorted((st[i], int(t.shape[i])) for i in range(4) if int(t.shape[i]) > 1)
    for (s0, n0), (s1, _) in zip(dims, dims[1:]):
        if s1 < s0 * n0:
            return "stride_overlap"
    return None


def torch_stream(device=None):
    return int(torch.cuda.current_stream(device).cuda_stream)


def _dtype_code(dt):
    if dt == torch.float16:
        return SAGE_F16
    if dt == torch.bfloat16:
        return SAGE_BF16
    raise ValueError("dtype: %s is not served (fp16 and bf16 only)" % dt)


def _ptr(t):
    return ctypes.c_void_p(0 if t is None else int(t.data_ptr()))


def hip_runtime_images():
    """The distinct HIP runtime files (`libamdhip64`) mapped into this process, or None where
    /proc/self/maps cannot be read. One image means the library and torch share the runtime (and
    so torch's stream handles are valid for the library's launches), which the reference records
    as its `same_as_torch` check (`sageattention/sk1_backend/sk1_loader.py:218-251`)."""
    try:
        with open("/proc/self/maps") as f:
            maps = f.read()
    except OSError:
        return None
    return sorted({ln.split()[-1] for ln in maps.splitlines() if "libamdhip64" in ln})


class SageLib:
    """The loaded library. `SageLib.get()` loads it once per process (under a lock) and raises
    `RuntimeError` when it is missing or does not load: there is no other backend to fall back to."""

    _instance = None
    _lock = threading.Lock()

    @classmethod
    def get(cls):
        if cls._instance is None:
            with cls._lock:
                if cls._instance is None:
                    cls._instance = cls(LIB_PATH)
        return cls._instance

    def __init__(self, path):
        if not os.path.isfile(path):
            raise RuntimeError(
                "the gfx950 library %s is not built (run `python sageattention-rdna4_amd/"
                "build_lib.py` or `__graft_entry__.build()`)" % path)
        self.path = path
        self.lib = ctypes.CDLL(path, mode=ctypes.RTLD_GLOBAL)
        L = self.lib
        i64, f32, vp, i32 = ctypes.c_int64, ctypes.c_float, ctypes.c_void_p, ctypes.c_int
        L.sage_version.restype = i32
        L.sage_version.argtypes = []
        L.sage_last_error.restype = ctypes.c_char_p
        L.sage_last_error.argtypes = []
        L.sage_build_id.restype = ctypes.c_char_p
        L.sage_build_id.argtypes = []
        L.sage_kv_prologue_workspace_bytes.restype = ctypes.c_size_t
        L.sage_kv_prologue_workspace_bytes.argtypes = [i64, i64]
        L.sage_kv_prologue.restype = i32
        L.sage_kv_prologue.argtypes = ([i32] * 5 + [vp, i64, i64, i64] * 2 + [i64] * 5
                                       + [vp] * 9 + [ctypes.c_size_t, vp])
        L.sage_kv_prologue_noalloc.restype = i32
        L.sage_kv_prologue_noalloc.argtypes = ([i32] * 5 + [vp, i64, i64, i64] * 2 + [i64] * 5
                                               + [vp] * 9)
        L.sage_attn_fwd.restype = i32
        L.sage_attn_fwd.argtypes = ([i32] * 3 + [vp, i64, i64, i64] + [vp] * 4
                                    + [vp, i64, i64, i64] + [i64] * 4 + [f32, vp])
        L.sage_attn_fwd_ex.restype = i32
        L.sage_attn_fwd_ex.argtypes = ([i32] * 3 + [vp, i64, i64, i64] + [vp] * 4
                                       + [vp, i64, i64, i64] + [i64] * 7
                                       + [f32, i32, vp, vp, vp, vp])
        L.sage_attn_fwd_sk.restype = i32
        L.sage_attn_fwd_sk.argtypes = ([i32] * 3 + [vp, i64, i64, i64] + [vp] * 6
                                       + [vp, i64, i64, i64] + [i64] * 7 + [f32, vp, vp, vp])
        L.sage_kseq_mean.restype = i32
        L.sage_kseq_mean.argtypes = [i32, vp, i64, i64, i64, i64, i64, i64, i64, vp, vp,
                                     ctypes.c_size_t, vp]
        L.sage_quant_q.restype = i32
        L.sage_quant_q.argtypes = [i32, i32, vp, i64, i64, i64, i64, i64, i64, i64, f32, vp, vp,
                                   vp, vp]
        L.sage_mfma_layout_probe.restype = i32
        L.sage_mfma_layout_probe.argtypes = [vp] * 7
        L.sage_mfma_peak_probe.restype = i32
        L.sage_mfma_peak_probe.argtypes = [i32, i64, i64, vp, vp]
        L.sage_attn_kernel_choice.restype = i32
        L.sage_attn_kernel_choice.argtypes = [i64, i64, i64, i64, i32, i64]
        self.version = int(L.sage_version())
        self.build_id = L.sage_build_id().decode()
        images = hip_runtime_images()
        self.hip_runtime = images
        self.same_as_torch = None if images is None else len(images) == 1

    # ------------------------------------------------------------------ helpers
    def _check(self, rc, what):
        if rc != 0:
            msg = self.lib.sage_last_error().decode(errors="replace")
            if rc == 1:
                raise ValueError("%s: %s" % (what, msg))
            raise RuntimeError("%s: %s" % (what, msg))

    def workspace_bytes(self, BH, N):
        return int(self.lib.sage_kv_prologue_workspace_bytes(int(BH), int(N)))

    def kernel_choice(self, B, H, N, D, causal, cus=0):
        """The main-loop kernel code (2: 256-query ping-pong, 3: pipelined, 4: key split) the
        library's automatic choice runs for this shape on `cus` compute units (0: the current
        device's; see `sage_attn_kernel_choice`)."""
        rc = int(self.lib.sage_attn_kernel_choice(int(B), int(H), int(N), int(D), int(bool(causal)),
                                                  int(cus)))
        if rc < 0:
            self._check(-rc, "sage_attn_kernel_choice")
        return rc

    # ------------------------------------------------------------------ entry points
    def kv_prologue(self, k, v, k8, sk, v8t, sv, s, mean, workspace, *, k_int8, smooth_k, fold,
                    n_pad, kconst=None, smooth_v=False, vmean=None):
        """K/V prologue on logical (B, H, N, D) views `k`, `v`, D = 64 or 128 (see
        `sage_kv_prologue`).
        `kconst` (optional) receives the main loop's per-key constants, (B*H, N_pad/64, 2, 64);
        with `smooth_v`, `vmean` ((B*H, 128) fp32) receives V's sequence mean."""
        B, H, N, D = (int(x) for x in k.shape)
        rc = self.lib.sage_kv_prologue(
            _dtype_code(k.dtype), int(bool(k_int8)), int(bool(smooth_k)), int(bool(smooth_v)),
            int(bool(fold)), _ptr(k), k.stride(0), k.stride(1), k.stride(2),
            _ptr(v), v.stride(0), v.stride(1), v.stride(2),
            B, H, N, int(n_pad), D, _ptr(k8), _ptr(sk), _ptr(v8t), _ptr(sv), _ptr(mean),
            _ptr(vmean), _ptr(s), _ptr(kconst), _ptr(workspace),
            int(workspace.numel() * workspace.element_size()),
            ctypes.c_void_p(torch_stream(k.device)))
        self._check(rc, "sage_kv_prologue")

    def prologue_and_main(self, q, k, v, o, base, off, ws_bytes, n_pad, *, qk_int8, smooth_k,
                          smooth_v, causal, sm_scale, kernel, lse, stream, events=None):
        """The served call's two library calls (`sage_kv_prologue`, then `sage_attn_fwd_ex`) on
        one device buffer that holds every temporary: K8, SK, V8T, SV, S, KCONST and the workspace
        (and KMEAN, VMEAN when present) at the byte offsets `off[name]` from address `base`.
        `q`, `o` are logical (B, H, N, D) views, `k`, `v` (B, H_kv, N_kv, D). One stream handle for
        both calls; `events` (three, optional) are recorded before, between and after them."""
        B, H, N, D = q.shape
        H_kv, N_kv = k.shape[1], k.shape[2]
        vp = ctypes.c_void_p

        def at(name):
            o_ = off.get(name)
            return None if o_ is None else vp(base + o_)

        dt = _dtype_code(q.dtype)
        st = vp(stream)
        ks, vs, qs, os_ = k.stride(), v.stride(), q.stride(), o.stride()
        if events is not None:
            events[0].record()
        rc = self.lib.sage_kv_prologue(
            dt, int(qk_int8), int(smooth_k), int(smooth_v), 1, vp(k.data_ptr()), ks[0], ks[1],
            ks[2], vp(v.data_ptr()), vs[0], vs[1], vs[2], B, H_kv, N_kv, n_pad, D, at("k8"),
            at("sk"), at("v8t"), at("sv"), at("kmean"), at("vmean"), at("s"), at("kconst"),
            at("ws"), ws_bytes, st)
        self._check(rc, "sage_kv_prologue")
        if events is not None:
            events[1].record()
        rc = self.lib.sage_attn_fwd_ex(
            dt, int(qk_int8), int(causal), vp(q.data_ptr()), qs[0], qs[1], qs[2], at("k8"),
            at("kconst"), at("v8t"), at("s"), vp(o.data_ptr()), os_[0], os_[1], os_[2], B, H, N,
            H_kv, N_kv, n_pad, D, ctypes.c_float(sm_scale), int(kernel), _ptr(lse), at("kmean"),
            at("vmean"), st)
        self._check(rc, "sage_attn_fwd")
        if events is not None:
            events[2].record()

    def kv_prologue_noalloc(self, k, v, k8, sk, v8t, sv, s, mean, *, k_int8, smooth_k, fold,
                            n_pad, kconst=None, smooth_v=False, vmean=None):
        """`kv_prologue` with the library's static per-GPU scratch as its workspace (see
        `sage_kv_prologue_noalloc`): nothing is allocated. Calls overlapping on one GPU race."""
        B, H, N, D = (int(x) for x in k.shape)
        rc = self.lib.sage_kv_prologue_noalloc(
            _dtype_code(k.dtype), int(bool(k_int8)), int(bool(smooth_k)), int(bool(smooth_v)),
            int(bool(fold)), _ptr(k), k.stride(0), k.stride(1), k.stride(2),
            _ptr(v), v.stride(0), v.stride(1), v.stride(2),
            B, H, N, int(n_pad), D, _ptr(k8), _ptr(sk), _ptr(v8t), _ptr(sv), _ptr(mean),
            _ptr(vmean), _ptr(s), _ptr(kconst), ctypes.c_void_p(torch_stream(k.device)))
        self._check(rc, "sage_kv_prologue_noalloc")

    def attn_fwd(self, q, k8, kconst, v8t, s, o, *, qk_int8, causal, sm_scale, n_pad, kernel=0,
                 lse=None, kmean=None, n_kv=None, vmean=None):
        """Main loop on logical (B, H, N, D) views `q`, `o` (see `sage_attn_fwd_ex`; `kernel`:
        0 the library's choice by grid fill, 1 the 128-query kernel, 2 the 256-query ping-pong,
        3 the pipelined 128-query kernel, 4 its key split for non-causal head_dim 64). The
        prologue outputs `k8` (B*H_kv, n_pad, D) etc. give H_kv; `n_kv` is the key count (default N, and `n_pad`
        is then ceil(n_kv/64)*64). `lse` (optional, (B, H, N) fp32) receives each row's
        logsumexp; `kmean` ((B*H_kv, 128) fp32) adds its smooth_k correction; `vmean`
        ((B*H_kv, 128) fp32, optional) is added to every output row (smooth_v)."""
        B, H, N, D = (int(x) for x in q.shape)
        bh_kv = int(k8.shape[0])
        if bh_kv % B:
            raise ValueError("sage_attn_fwd: k8 holds %d planes, not a multiple of B=%d" % (bh_kv, B))
        n_kv = N if n_kv is None else int(n_kv)
        rc = self.lib.sage_attn_fwd_ex(
            _dtype_code(q.dtype), int(bool(qk_int8)), int(bool(causal)),
            _ptr(q), q.stride(0), q.stride(1), q.stride(2),
            _ptr(k8), _ptr(kconst), _ptr(v8t), _ptr(s),
            _ptr(o), o.stride(0), o.stride(1), o.stride(2),
            B, H, N, bh_kv // B, n_kv, int(n_pad), D, ctypes.c_float(float(sm_scale)), int(kernel),
            _ptr(lse), _ptr(kmean), _ptr(vmean), ctypes.c_void_p(torch_stream(q.device)))
        self._check(rc, "sage_attn_fwd")

    def attn_fwd_sk(self, q, k8, sk, v8t, sv, s, o, *, qk_int8, causal, sm_scale, n_kv=None,
                    vmean=None, lse=None, kmean=None):
        """Main loop on the reference kernel's inputs (see `sage_attn_fwd_sk`): `sk`, `sv`
        (B*H_kv, n_pad) fp32 are SK and the folded SV'; `s` (B*H_kv,) the fold."""
        B, H, N, D = (int(x) for x in q.shape)
        bh_kv, n_pad = int(k8.shape[0]), int(k8.shape[1])
        if bh_kv % B:
            raise ValueError("sage_attn_fwd_sk: k8 holds %d planes, not a multiple of B=%d"
                             % (bh_kv, B))
        n_kv = N if n_kv is None else int(n_kv)
        rc = self.lib.sage_attn_fwd_sk(
            _dtype_code(q.dtype), int(bool(qk_int8)), int(bool(causal)),
            _ptr(q), q.stride(0), q.stride(1), q.stride(2),
            _ptr(k8), _ptr(sk), _ptr(v8t), _ptr(sv), _ptr(vmean), _ptr(s),
            _ptr(o), o.stride(0), o.stride(1), o.stride(2),
            B, H, N, bh_kv // B, n_kv, n_pad, D, ctypes.c_float(float(sm_scale)),
            _ptr(lse), _ptr(kmean), ctypes.c_void_p(torch_stream(q.device)))
        self._check(rc, "sage_attn_fwd_sk")

    def kseq_mean(self, k, mean, workspace):
        """The smooth_k mean of a logical (B, H, N, D) view into `mean` (B*H, D) fp32 (see
        `sage_kseq_mean`)."""
        B, H, N, D = (int(x) for x in k.shape)
        rc = self.lib.sage_kseq_mean(
            _dtype_code(k.dtype), _ptr(k), k.stride(0), k.stride(1), k.stride(2), B, H, N, D,
            _ptr(mean), _ptr(workspace), int(workspace.numel() * workspace.element_size()),
            ctypes.c_void_p(torch_stream(k.device)))
        self._check(rc, "sage_kseq_mean")

    def quant_q(self, q, sm_scale, *, qk_int8):
        """Q quantized exactly as the main loop quantizes it: `(q8, sq, cq)` on q's device."""
        B, H, N, D = (int(x) for x in q.shape)
        dev = q.device
        q8 = torch.empty(B * H, N, D, device=dev,
                         dtype=torch.int8 if qk_int8 else torch.float8_e4m3fn)
        sq = torch.empty(B * H, N, device=dev, dtype=torch.float32)
        cq = torch.empty(B * H, N, device=dev, dtype=torch.float32)
        rc = self.lib.sage_quant_q(
            _dtype_code(q.dtype), int(bool(qk_int8)), _ptr(q), q.stride(0), q.stride(1),
            q.stride(2), B, H, N, D, ctypes.c_float(float(sm_scale)), _ptr(q8), _ptr(sq), _ptr(cq),
            ctypes.c_void_p(torch_stream(dev)))
        self._check(rc, "sage_quant_q")
        return q8, sq, cq

    #: MFMAs per wave per round of `sage_mfma_peak_probe`, and waves per block
    PEAK_NACC, PEAK_WAVES = 4, 4

    def mfma_peak_probe(self, qk_int8, blocks, iters, clocks=None, device=None):
        """Launch the MFMA throughput probe on the current stream of `device`; returns its op
        count (see `sage_mfma_peak_probe`). `clocks` (optional, 2 int64 on the device) receives
        the first wave's shader-clock cycles and constant-rate ticks."""
        rc = self.lib.sage_mfma_peak_probe(int(bool(qk_int8)), int(blocks), int(iters),
                                           _ptr(clocks), ctypes.c_void_p(torch_stream(device)))
        self._check(rc, "sage_mfma_peak_probe")
        k = 32 if qk_int8 else 64
        return int(blocks) * self.PEAK_WAVES * int(iters) * self.PEAK_NACC * 2 * 32 * 32 * k

    def layout_probe(self, a, bt, e, ft):
        dev = a.device
        c = torch.empty(32, 32, device=dev, dtype=torch.int32)
        d = torch.empty(32, 32, device=dev, dtype=torch.float32)
        rc = self.lib.sage_mfma_layout_probe(_ptr(a), _ptr(bt), _ptr(c), _ptr(e), _ptr(ft), _ptr(d),
                                             ctypes.c_void_p(torch_stream(dev)))
        self._check(rc, "sage_mfma_layout_probe")
        return c, d
