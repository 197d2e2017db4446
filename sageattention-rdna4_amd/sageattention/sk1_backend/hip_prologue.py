"""The K/V prologue: the reference's `HipPrologue` interface over the gfx950 library.

Mirrors `sageattention/sk1_backend/hip_prologue.py` of the reference: `n_pad_for`, the refusal
vocabulary `REFUSALS`, `check`, `quant_kv` (returns `(k8, sk, v8t, sv)` freshly allocated, or
`None` on a refusal and never raises) and `kseq_mean`. Differences, all from this build's design:

* the mean, the K/V quantization and the per-(b,h) V-scale fold run as two launches of one library
  call; `quant_kv(..., fold=True)` also returns `S` and leaves `SV' = SV/S` in `sv` (the reference
  runs `fold_v_scale`, three torch ops, afterwards: `sk1_backend/__init__.py:561-579`);
* head_dim is 64 or 128, as the reference's (its D=64 prologue feeds no served kernel there;
  here the 128-query main loop serves D=64);
* `floor` is fixed at the reference's 1e-12.
"""
import collections

import torch

from .sk1_loader import STRIDED_REFUSALS, SageLib, strided_view_reason

HEAD_DIMS = (64, 128)
BN = 64
FLOOR = 1e-12

#: every reason `check` / `quant_kv` / `kseq_mean` can return, so a test can enumerate them
REFUSALS = ("not_cuda", "rank", "shape", "dtype_mismatch", "bf16_int8", "dtype", "head_dim",
            "device", "n_pad", "n_lt_1", "floor", "launch", "mean_dtype", "mean_head_dim",
            "mean_launch") + tuple(
    p + r for p in ("k_", "v_", "mean_") for r in STRIDED_REFUSALS)


def n_pad_for(N: int) -> int:
    """SK1's N_pad contract: a multiple of 64 (`hip_prologue.py:93-95` of the reference)."""
    return ((int(N) + BN - 1) // BN) * BN


class HipPrologue:
    """The prologue entry points. One instance per process (`get()`); raises at construction when
    the library is missing."""

    _inst = None

    @classmethod
    def get(cls):
        if cls._inst is None:
            cls._inst = cls()
        return cls._inst

    def __init__(self, lib=None):
        self.lib = lib if lib is not None else SageLib.get()
        self.n_calls = 0
        self.n_refusals = 0
        self.refusal_reasons = collections.Counter()
        self.last_error = None

    def describe(self):
        return "%s (version %d)" % (self.lib.path, self.lib.version)

    def check(self, k, v, n_pad, int8):
        """`None` if this call is inside the prologue's contract, else a reason string
        (`hip_prologue.py:145-185` of the reference)."""
        if not (k.is_cuda and v.is_cuda):
            return "not_cuda"
        if k.dim() != 4 or v.dim() != 4:
            return "rank"
        if tuple(k.shape) != tuple(v.shape):
            return "shape"
        if k.dtype != v.dtype:
            return "dtype_mismatch"
        if k.dtype == torch.bfloat16:
            if int8:
                return "bf16_int8"
        elif k.dtype != torch.float16:
            return "dtype"
        if int(k.shape[3]) not in HEAD_DIMS:
            return "head_dim"
        if k.device != v.device:
            return "device"
        r = strided_view_reason(k, "k")
        if r is not None:
            return "k_" + r
        r = strided_view_reason(v, "v")
        if r is not None:
            return "v_" + r
        N = int(k.shape[2])
        if N < 1:
            return "n_lt_1"
        if int(n_pad) < N or int(n_pad) % BN:
            return "n_pad"
        return None

    def quant_kv(self, k, v, n_pad=None, smooth_k=False, int8=True, floor=FLOOR, fold=False,
                 mean_out=False):
        """`(k8, sk, v8t, sv)` for logical (B, H, N, D) fp16/bf16 `k`/`v` (D = 64 or 128), or
        `None` if refused.

        With `fold=True` the tuple gains `S` (B*H,) and `sv` holds `SV' = SV / S`. With
        `mean_out=True` (and smooth_k) the tuple also gains the mean (B*H, D). Never raises: a
        refusal or a launch error returns `None` and is counted in `refusal_reasons`.
        """
        if k.dim() != 4 or v.dim() != 4:
            return self._refuse("rank")
        B, H, N, D = (int(x) for x in k.shape)
        BH = B * H
        n_pad = n_pad_for(N) if n_pad is None else int(n_pad)
        reason = self.check(k, v, n_pad, int8)
        if reason is not None:
            return self._refuse(reason)
        if float(floor) != FLOOR:
            return self._refuse("floor")
        dev = k.device
        try:
            k8 = torch.empty(BH, n_pad, D, device=dev,
                             dtype=torch.int8 if int8 else torch.float8_e4m3fn)
            sk = torch.empty(BH, n_pad, device=dev, dtype=torch.float32)
            v8t = torch.empty(BH, D, n_pad, device=dev, dtype=torch.float8_e4m3fn)
            sv = torch.empty(BH, n_pad, device=dev, dtype=torch.float32)
            s = torch.empty(BH, device=dev, dtype=torch.float32)
            mean = torch.empty(BH, D, device=dev, dtype=torch.float32) if smooth_k else None
            ws = torch.empty(self.lib.workspace_bytes(BH, N), device=dev, dtype=torch.uint8)
            with torch.cuda.device(dev):
                self.lib.kv_prologue(k, v, k8, sk, v8t, sv, s, mean, ws, k_int8=int8,
                                     smooth_k=smooth_k, fold=fold, n_pad=n_pad)
        except Exception as e:  # noqa: BLE001 - the reference's prologue contract is "never raises"
            self.last_error = "%s: %s" % (type(e).__name__, e)
            return self._refuse("launch")
        self.n_calls += 1
        res = (k8, sk, v8t, sv)
        if fold:
            res = res + (s,)
        if mean_out and smooth_k:
            res = res + (mean,)
        return res

    def kseq_mean(self, k):
        """The smooth_k sequence mean (B, H, D) fp32, or `None` if refused (never raises).

        fp64 sums of the exactly widened inputs in a fixed order, one fp32 rounding: the same bits
        as the `mean` the prologue subtracts (`hip_prologue.py:267-292` of the reference, whose
        kernel is `h34_kseq_mean_*`). K is read once; V is not read.
        """
        if k.dim() != 4 or not k.is_cuda or k.dtype not in (torch.float16, torch.bfloat16):
            return self._refuse("mean_dtype")
        B, H, N, D = (int(x) for x in k.shape)
        if D not in HEAD_DIMS:
            return self._refuse("mean_head_dim")
        r = strided_view_reason(k, "k")
        if r is not None:
            return self._refuse("mean_" + r)
        if N < 1:
            return self._refuse("n_lt_1")
        try:
            mean = torch.empty(B * H, D, device=k.device, dtype=torch.float32)
            ws = torch.empty(self.lib.workspace_bytes(B * H, N), device=k.device,
                             dtype=torch.uint8)
            with torch.cuda.device(k.device):
                self.lib.kseq_mean(k, mean, ws)
        except Exception as e:  # noqa: BLE001 - the reference's prologue contract is "never raises"
            self.last_error = "%s: %s" % (type(e).__name__, e)
            return self._refuse("mean_launch")
        self.n_calls += 1
        return mean.view(B, H, D)

    def _refuse(self, reason):
        self.n_refusals += 1
        self.refusal_reasons[reason] += 1
        return None
