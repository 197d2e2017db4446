"""The SK1 router on MI355X: envelope check, prologue, main loop.

Mirrors `sageattention/sk1_backend/__init__.py` of the reference (`ENVELOPE` `:346-358`,
`_envelope_ok` `:920-979`, `try_sk1_t1` `:982-1284`), re-designed for one backend:

* one library (`libsagemi355.so`, gfx950) serves every call inside the envelope; there is no
  fallback chain, no code-object selection and no backend switch;
* fp16 inputs run int8 Q.K (the reference's `sk1_t6i`/`sk1_t6in`), bf16 inputs fp8 Q.K (the
  reference's `sk1_t4a1sb`/`sk1_t4a1nb`); `int8=False` forces fp8 Q.K for fp16 inputs (the
  reference's fp8 fp16 object), for comparisons;
* contiguous HND, NHD and any other view the stride rule accepts take the same kernel (strides are
  arguments), so NHD and fused-QKV views give the same bits as contiguous HND;
* the per-(b,h) V-scale fold runs inside the prologue launch pair, not as three torch ops.

`try_sk1_t1` keeps the reference's contract: `(out, None)` when served, `(None, reason)` when the
call is outside the envelope or (with `strict=False`) when the library fails.
"""
import sys
from contextlib import nullcontext

import torch

from .hip_prologue import HipPrologue, n_pad_for  # noqa: F401
from .sk1_loader import (STRIDED_REFUSALS, SageLib, strided_view_reason,  # noqa: F401
                         torch_stream)

#: The architectures the library is built for.
SUPPORTED_ARCHS = ("gfx950",)

#: What this build serves. `layout` HND or NHD; `contiguous` = any view `strided_view_reason`
#: accepts (contiguous HND, physically-NHD, fused-QKV splits); head_dim 64 or 128.
ENVELOPE = dict(
    layout=("HND", "NHD"),
    dtype=("fp16", "bf16"),
    head_dim=(64, 128),
    contiguous="any view strided_view_reason accepts",
    causal=(0, 1),
    smooth_k=(False, True),
    batch_heads=("any B*H whose grids fit HIP's 2^32-1 threads per launch: "
                 "B*H*ceil(N/128) < 2^24, B*H*ceil(N/256) < 2^23, B*H < 2^24"),
    heads="H_kv divides H (grouped-query / multi-query K/V heads)",
    seq_len="N >= 1, N_kv >= 1; N == N_kv when causal",
    return_lse=(False, True),
    attn_mask=False,
    smooth_v=(False, True),
)

_LOGGED = set()


def _log_once(msg):
    if msg not in _LOGGED:
        _LOGGED.add(msg)
        print("[sageattention-mi355] %s" % msg, file=sys.stderr)


def device_arch(device=None) -> str:
    """The device's `gcnArchName` prefix (before `:`), or "" if it cannot be read. Never raises.

    A named module function so a test can monkeypatch the arch query
    (`sageattention/sk1_backend/__init__.py:393-410` of the reference).
    """
    try:
        if device is None:
            device = torch.cuda.current_device()
        name = getattr(torch.cuda.get_device_properties(device), "gcnArchName", "") or ""
        return name.split(":", 1)[0]
    except Exception:  # noqa: BLE001
        return ""


def arch_supported(device=None) -> bool:
    return globals()["device_arch"](device) in SUPPORTED_ARCHS


def _envelope_ok(q, k, v, tensor_layout, is_causal, sm_scale, return_lse, smooth_k, smooth_v,
                 attn_mask):
    """`None` when the call is served, else the refusal reason (the reference's strings,
    `sageattention/sk1_backend/__init__.py:920-979`)."""
    if tensor_layout not in ("HND", "NHD"):
        return "layout"
    if attn_mask is not None:
        return "attn_mask"
    if not (isinstance(q, torch.Tensor) and isinstance(k, torch.Tensor)
            and isinstance(v, torch.Tensor)):
        return "device"
    if not (q.is_cuda and k.is_cuda and v.is_cuda):
        return "device"
    if q.device != k.device or q.device != v.device:
        return "device"
    if not (q.dtype == k.dtype == v.dtype):
        return "dtype"
    if q.dtype not in (torch.float16, torch.bfloat16):
        return "dtype"
    if not (q.dim() == 4 and k.dim() == 4 and v.dim() == 4):
        return "rank"
    if tensor_layout == "NHD":
        q, k, v = q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2)
    for nm, t in (("q", q), ("k", k), ("v", v)):
        r = strided_view_reason(t, nm)
        if r is not None:
            return r
    # head_dim 64 or 128, the three tensors agreeing (the reference's rule, `__init__.py:962-965`;
    # its D=64 object is never routed, `:208-229`; here the 128-query main loop serves it)
    if q.size(3) not in (64, 128) or k.size(3) != q.size(3) or v.size(3) != q.size(3):
        return "head_dim"
    if q.size(0) != k.size(0) or q.size(0) != v.size(0):
        return "batch"
    # grouped K/V heads and a key length of its own, as the upstream API allows them
    # (`sageattention/core.py:824-829` of the reference; its SK1 envelope refuses both,
    # `sk1_backend/__init__.py:966-978`): H a multiple of H_kv, causal only with N == N_kv
    if k.size(1) != v.size(1) or k.size(1) < 1 or q.size(1) % k.size(1) != 0:
        return "heads"
    if k.size(2) != v.size(2):
        return "seq_len"
    if q.size(2) < 1 or k.size(2) < 1:
        return "seq_len"
    if is_causal and q.size(2) != k.size(2):
        return "seq_len"
    return None


def try_sk1_t1(q, k, v, *, tensor_layout="HND", is_causal=False, sm_scale=None, return_lse=False,
               smooth_k=True, smooth_v=False, attn_mask=None, strict=False, int8=None, bf16=None):
    """Run the gfx950 SK1 path if the call is inside `ENVELOPE`.

    Returns `(out, None)` with `out` in the caller's layout and dtype (`(out, lse)` as `out` with
    `return_lse=True`, lse (B, H, N) fp32), or `(None, reason)`.
    `strict=True` raises instead of returning a refusal for a wrong arch or a library failure
    (envelope misses are always returned as a reason). `int8=False` selects fp8 Q.K for fp16
    inputs; `bf16` is accepted for signature compatibility (bf16 is always served).
    """
    del bf16
    reason = _envelope_ok(q, k, v, tensor_layout, is_causal, sm_scale, return_lse, smooth_k,
                          smooth_v, attn_mask)
    if reason is not None:
        return None, reason
    if not arch_supported(q.device):
        msg = ("device arch is %r; libsagemi355.so is built for %s"
               % (device_arch(q.device) or "<unknown>", ", ".join(SUPPORTED_ARCHS)))
        if strict:
            raise RuntimeError(msg)
        _log_once(msg)
        return None, "arch"
    try:
        lib = SageLib.get()
    except Exception as e:
        if strict:
            raise
        _log_once("load failed: %s" % e)
        return None, "load_failed"

    try:
        out = sk1_forward(lib, q, k, v, tensor_layout=tensor_layout, is_causal=is_causal,
                          sm_scale=sm_scale, smooth_k=smooth_k, int8=int8,
                          return_lse=bool(return_lse), smooth_v=bool(smooth_v))
    except Exception as e:
        if strict:
            raise
        _log_once("launch failed: %s" % e)
        return None, "launch_failed"
    return out, None


def sk1_forward(lib, q, k, v, *, tensor_layout="HND", is_causal=False, sm_scale=None,
                smooth_k=True, int8=None, events=None, kernel=0, return_lse=False,
                smooth_v=False):
    """The served path without the envelope check: allocate, prologue (2 launches), main loop.
    q is (B, H, N, D) and k, v (B, H_kv, N_kv, D) in HND terms: query head h reads K/V head
    h // (H // H_kv); N may differ from N_kv when not causal. `smooth_v` subtracts V's sequence
    mean before quantizing V and adds it back to the output (exact, since each row's weights sum
    to 1; the reference's `quant_triton.py:668-678`).
    `kernel` picks the main-loop kernel (0: the library's choice by grid fill, 1: 128 queries per
    block, 2: 256, head_dim 128 only, 3: the pipelined 128-query kernel, 4: its key split,
    non-causal head_dim 64 only: the same probabilities as 1-3, its fp32 sums rounded in another
    order).
    With `return_lse`, returns `(out, lse)`: lse (B, H, N) fp32, each row's natural-log
    logsumexp of its scores times sm_scale (with smooth_k, corrected by sm_scale * q . mean_k, as
    the reference's `core.py:1437-1439`).

    `events`, when given, is a sequence of three `torch.cuda.Event`s recorded on the launch stream
    before the prologue, between the prologue and the main loop, and after the main loop.
    """
    if tensor_layout == "NHD":
        qq, kk, vv = q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2)
    else:
        qq, kk, vv = q, k, v
    B, H, N, D = (int(x) for x in qq.shape)
    H_kv, N_kv = int(kk.shape[1]), int(kk.shape[2])
    BH_kv = B * H_kv
    is_bf16 = q.dtype == torch.bfloat16
    qk_int8 = (not is_bf16) and (int8 is None or bool(int8))
    sm = float(sm_scale if sm_scale is not None else D ** -0.5)
    n_pad = n_pad_for(N_kv)
    dev = q.device
    # Every temporary of the call in one allocation, 256-byte aligned parts: the prologue's
    # outputs per K/V plane (B*H_kv planes of N_kv keys) -- K8, SK, V8T, SV, S, KCONST -- its
    # workspace, and K's mean (for the logsumexp) and V's mean (smooth_v) when used.
    el8, nf = BH_kv * n_pad * D, BH_kv * n_pad * 4
    ws_bytes = lib.workspace_bytes(BH_kv, N_kv)
    parts = [("k8", el8), ("sk", nf), ("v8t", el8), ("sv", nf), ("s", BH_kv * 4),
             ("kconst", 2 * nf), ("ws", ws_bytes)]
    if return_lse and smooth_k:
        parts.append(("kmean", BH_kv * D * 4))
    if smooth_v:
        parts.append(("vmean", BH_kv * D * 4))
    off, total = {}, 0
    for name, nbytes in parts:
        off[name] = total
        total += (nbytes + 255) // 256 * 256
    tmp = torch.empty(total, device=dev, dtype=torch.uint8)
    lse = torch.empty(B, H, N, device=dev, dtype=torch.float32) if return_lse else None
    if tensor_layout == "NHD":
        out = torch.empty(B, N, H, D, device=dev, dtype=q.dtype)
        oo = out.transpose(1, 2)
    else:
        out = torch.empty(B, H, N, D, device=dev, dtype=q.dtype)
        oo = out
    ctx = torch.cuda.device(dev) if dev.index != torch.cuda.current_device() else nullcontext()
    with ctx:
        lib.prologue_and_main(qq, kk, vv, oo, tmp.data_ptr(), off, ws_bytes, n_pad,
                              qk_int8=qk_int8, smooth_k=bool(smooth_k), smooth_v=bool(smooth_v),
                              causal=bool(is_causal), sm_scale=sm, kernel=kernel, lse=lse,
                              stream=torch_stream(dev), events=events)
    return (out, lse) if return_lse else out
