"""`sageattn`: the drop-in entry point of the quantized attention path.

Same name and signature as the reference's dispatcher (`sageattention/core.py:1037-1049`):
`sageattn(q, k, v, tensor_layout="HND", is_causal=False, sm_scale=None, return_lse=False,
sk1_backend=None, sk1_int8=None, sk1_bf16=None, **kwargs)`, with `smooth_k` (default True),
`smooth_v` and `attn_mask` arriving through kwargs (`core.py:1162`, `:1198-1207`).

There is exactly one backend here, the gfx950 library. A call outside its envelope raises a clear
error instead of silently falling back (the reference falls back to its PR #368 path): `attn_mask`
raises `NotImplementedError` as in `core.py:1156-1161`; any other miss (head_dim not 64 or 128,
H not a multiple of H_kv, causal with q_len != kv_len, other dtypes) raises `ValueError` naming
the reason. `return_lse=True` returns `(out, lse)` with lse (B, H, N) fp32 as the reference's
`core.py:1081-1095` defines it; grouped K/V heads and a key length of their own are served as the
upstream API serves them (`core.py:824-829`); `smooth_v=True` subtracts V's sequence mean before
quantizing V and adds it back to the output (`core.py:395-421`; in the SK1 scheme the reference's
`quant_triton.py:668-678` with the VMEAN epilogue of `kernels/hip/sk1_t6i.hip:290-297`). The
reference's SK1 path refuses all four.
"""
from .sk1_backend import try_sk1_t1

#: kwargs of the reference's signature that this build accepts and ignores: they select
#: quantization granularity / accumulation variants of the PR #368 fallback path.
_IGNORED_KWARGS = ("qk_quant_gran", "pv_accum_dtype", "value_dtype")


def sageattn(q, k, v, tensor_layout="HND", is_causal=False, sm_scale=None, return_lse=False,
             sk1_backend=None, sk1_int8=None, sk1_bf16=None, **kwargs):
    """Quantized self-attention: int8 (fp16 inputs) or fp8 (bf16 inputs) Q.K, fp8 P.V.

    q: (B, H, N, D) for `tensor_layout="HND"` or (B, N, H, D) for "NHD", D = 64 or 128; k, v
    likewise with H_kv heads (H a multiple of H_kv: query head h reads K/V head h // (H // H_kv))
    and N_kv rows (N_kv == N when causal); fp16 or bf16, on a gfx950 device. Returns the output in
    q's layout and dtype; with `return_lse=True`, the pair `(out, lse)`, lse (B, H, N) fp32: the natural-log
    logsumexp of each row of Q.K^T * sm_scale.
    kwargs: `smooth_k` (default True) subtracts the sequence mean of K before quantizing it;
    `smooth_v` (default False) subtracts V's and adds it back to the output.
    `sk1_int8=False` selects fp8 Q.K for fp16 inputs; `sk1_backend` and `sk1_bf16` are accepted and
    ignored (there is one backend).
    """
    del sk1_backend
    attn_mask = kwargs.pop("attn_mask", None)
    if attn_mask is not None:
        raise NotImplementedError("sageattn does not support attn_mask")
    smooth_k = kwargs.pop("smooth_k", True)
    smooth_v = kwargs.pop("smooth_v", False)
    for name in _IGNORED_KWARGS:
        kwargs.pop(name, None)
    if kwargs:
        raise TypeError("sageattn got unexpected keyword arguments: %s" % sorted(kwargs))
    out, reason = try_sk1_t1(q, k, v, tensor_layout=tensor_layout, is_causal=is_causal,
                             sm_scale=sm_scale, return_lse=return_lse, smooth_k=smooth_k,
                             smooth_v=smooth_v, attn_mask=None, strict=True, int8=sk1_int8,
                             bf16=sk1_bf16)
    if out is None:
        raise ValueError("sageattn: this call is outside the MI355X SK1 envelope (%s); see "
                         "sageattention.sk1_backend.ENVELOPE" % reason)
    return out
