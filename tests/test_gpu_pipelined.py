"""The software-pipelined main loop (SAGE_KERNEL_PIPE, attn_fwd_pl.hip) against the 128-query
kernel and the oracle (GPU).

Both kernels compute every score, row sum and accumulator update with the same operations on the
same values; only the order in which each wave issues its matrix work differs. So they must agree
bit for bit: outputs, logsumexp rows and smooth_v outputs, at lengths that exercise the pipeline's
edges (one block, the first and last blocks of a causal diagonal, ragged tails, the three-buffer
ring's wrap) for both dtypes and both head dims, and with grouped K/V heads.
"""
import pytest
import torch

import oracle
from sage_testutil import cosine, have_gfx950, make_qkv, rel_l1, rel_l1_bar

pytestmark = [pytest.mark.gpu,
              pytest.mark.skipif(not have_gfx950(), reason="needs a gfx950 GPU")]

PIPE, Q128 = 3, 1


def _run(q, k, v, *, causal, kernel, layout="HND", **kw):
    from sageattention.sk1_backend import sk1_forward
    from sageattention.sk1_backend.sk1_loader import SageLib
    out = sk1_forward(SageLib.get(), q.cuda(), k.cuda(), v.cuda(), tensor_layout=layout,
                      is_causal=causal, kernel=kernel, **kw)
    torch.cuda.synchronize()
    if isinstance(out, tuple):
        return tuple(t.cpu() for t in out)
    return out.cpu()


@pytest.mark.parametrize("D", [128, 64])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("N", [1, 63, 64, 65, 127, 129, 192, 255, 257, 511, 700, 1025, 2049])
def test_pipelined_equals_q128_bitwise(N, causal, dtype, D):
    print("case N", N, causal, dtype, D, flush=True)
    q, k, v = make_qkv(1, 3, N, seed=N + 5, dtype=dtype, k_offset_std=2.0, outlier_frac=0.01, d=D)
    o1 = _run(q, k, v, causal=causal, kernel=Q128)
    o3 = _run(q, k, v, causal=causal, kernel=PIPE)
    assert torch.equal(o1, o3), (o1.float() - o3.float()).abs().max().item()


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("causal", [False, True])
def test_pipelined_matches_emulation(causal, dtype):
    q, k, v = make_qkv(2, 2, 1337, seed=11, dtype=dtype, k_offset_std=2.0, outlier_frac=0.001)
    ref = oracle.emulate_sageattn(q, k, v, tensor_layout="HND", is_causal=causal)["o"]
    out = _run(q, k, v, causal=causal, kernel=PIPE)
    assert cosine(out, ref) >= 0.999 and rel_l1(out, ref) <= rel_l1_bar(dtype == torch.float16)


GQA_SHAPES = [
    # (B, H, H_kv, N, N_kv, causal)
    (1, 4, 2, 300, 300, True),
    (2, 6, 1, 130, 130, True),
    (1, 4, 4, 70, 1000, False),
    (1, 8, 2, 1000, 77, False),
    (1, 2, 1, 1, 300, False),
    (1, 3, 3, 257, 1, False),
    (2, 4, 2, 513, 1337, False),
]


@pytest.mark.parametrize("shape", GQA_SHAPES, ids=lambda s: "B%dH%dkv%dN%dNk%d%s" % (
    s[0], s[1], s[2], s[3], s[4], "c" if s[5] else ""))
def test_pipelined_gqa_lse_smooth_v_bitwise(shape):
    B, H, H_kv, N, N_kv, causal = shape
    q, k, v = make_qkv(B, H, N, seed=3 * N + N_kv, dtype=torch.float16, k_offset_std=2.0,
                       h_kv=H_kv, n_kv=N_kv, v_offset_std=1.0)
    for kw in ({}, {"return_lse": True}, {"smooth_v": True, "return_lse": True}):
        r1 = _run(q, k, v, causal=causal, kernel=Q128, **kw)
        r3 = _run(q, k, v, causal=causal, kernel=PIPE, **kw)
        r1 = r1 if isinstance(r1, tuple) else (r1,)
        r3 = r3 if isinstance(r3, tuple) else (r3,)
        for a, b in zip(r1, r3):
            assert torch.equal(a, b), (kw, (a.float() - b.float()).abs().max().item())


def test_pipelined_nhd_equals_hnd_bitwise():
    q, k, v = make_qkv(2, 3, 777, seed=3, dtype=torch.float16, layout="NHD")
    o_nhd = _run(q, k, v, causal=True, kernel=PIPE, layout="NHD")
    hnd = [t.transpose(1, 2).contiguous() for t in (q, k, v)]
    o_hnd = _run(*hnd, causal=True, kernel=PIPE)
    assert torch.equal(o_nhd.transpose(1, 2), o_hnd)
