"""A seeded sweep of random call shapes through the served path (GPU).

Each case draws batch, heads, K/V heads (GQA/MQA), query and key lengths, head_dim, dtype, layout,
causality, smooth_k, smooth_v and return_lse, then checks:
* `sageattn` against the CPU emulation of the reference scheme (cosine >= 0.999, rel-L1 <= 1e-2;
  the logsumexp rows within the bound of tests/test_gpu_attention.py);
* the main-loop kernels that serve the shape with the same arithmetic (128-query, pipelined, and
  the 256-query ping-pong at head_dim 128) bit for bit against each other, the key split
  (non-causal head_dim 64) against the same emulation, and the call `sageattn` served bit for bit
  against the kernel `sage_attn_kernel_choice` names.
The draws are fixed by the case seed, so a failure names a reproducible shape.
"""
import random

import pytest
import torch

import oracle
from sage_testutil import cosine, have_gfx950, make_qkv, rel_l1, rel_l1_bar

pytestmark = [pytest.mark.gpu,
              pytest.mark.skipif(not have_gfx950(), reason="needs a gfx950 GPU")]

N_CASES = 200


def _draw(seed):
    r = random.Random(seed)
    D = r.choice([64, 128, 128])
    dtype = r.choice([torch.float16, torch.float16, torch.bfloat16])
    causal = r.random() < 0.5
    B = r.choice([1, 1, 2, 3])
    H_kv = r.choice([1, 2, 3, 4])
    H = H_kv * r.choice([1, 1, 2, 3])
    N = r.choice([1, 2, 31, 64, 65, 100, 127, 200, 256, 257, 383, 500, 777, 1030, 1600])
    N_kv = N if causal else r.choice([N, 1, 63, 64, 65, 129, 300, 1111])
    layout = r.choice(["HND", "NHD"])
    smooth_k = r.random() < 0.8
    smooth_v = r.random() < 0.3
    lse = r.random() < 0.4
    k_off = r.choice([0.0, 2.0])
    outl = r.choice([0.0, 0.01])
    return dict(D=D, dtype=dtype, causal=causal, B=B, H=H, H_kv=H_kv, N=N, N_kv=N_kv,
                layout=layout, smooth_k=smooth_k, smooth_v=smooth_v, lse=lse, k_off=k_off,
                outl=outl)


@pytest.mark.parametrize("seed", range(N_CASES))
def test_random_shape(seed):
    from sageattention import sageattn
    from sageattention.sk1_backend import sk1_forward
    from sageattention.sk1_backend.sk1_loader import SageLib
    c = _draw(1000 + seed)
    print("case", seed, c, flush=True)
    q, k, v = make_qkv(c["B"], c["H"], c["N"], seed=seed, dtype=c["dtype"], layout=c["layout"],
                       k_offset_std=c["k_off"], outlier_frac=c["outl"], d=c["D"], h_kv=c["H_kv"],
                       n_kv=c["N_kv"], v_offset_std=1.0 if c["smooth_v"] else 0.0)
    kw = dict(tensor_layout=c["layout"], is_causal=c["causal"])
    res = sageattn(q.cuda(), k.cuda(), v.cuda(), return_lse=c["lse"], smooth_k=c["smooth_k"],
                   smooth_v=c["smooth_v"], **kw)
    torch.cuda.synchronize()
    out, lse = (res if c["lse"] else (res, None))
    out = out.cpu()
    em = oracle.emulate_sageattn(q, k, v, smooth_k=c["smooth_k"], smooth_v=c["smooth_v"], **kw)

    def check(out, lse):
        assert torch.isfinite(out).all()
        cs, rl = cosine(out, em["o"]), rel_l1(out, em["o"])
        assert cs >= 0.999 and rl <= rel_l1_bar(c["dtype"] == torch.float16), (cs, rl)
        if c["lse"]:
            lse = lse.cpu().double()
            ref = em["lse"].double()
            # the emulation's logsumexp up to 1e-3 + 1e-4 |lse|, plus the fp8 Q.K score error
            # bound of tests/test_gpu_attention.py when Q.K is fp8 (bf16 inputs)
            tol = 1e-3 + 1e-4 * ref.abs()
            if c["dtype"] == torch.bfloat16:
                sk = em["sk"].amax().item()
                cq = em["c_q"].view_as(ref).double()
                tol = tol + 2.0 ** -10 * 448 ** 2 * cq * sk / float(oracle.LOG2E)
            assert ((lse - ref).abs() <= tol).all(), (lse - ref).abs().max().item()

    check(out, lse)
    # the kernels 1-3 that serve the shape give the same bits; the key split (non-causal
    # head_dim 64) passes the same emulation check; the served call is the chosen kernel's
    lib = SageLib.get()
    kernels = [1, 3] + ([2] if c["D"] == 128 else []) + (
        [4] if c["D"] == 64 and not c["causal"] else [])
    outs = {}
    for kern in kernels:
        r = sk1_forward(lib, q.cuda(), k.cuda(), v.cuda(), smooth_k=c["smooth_k"],
                        smooth_v=c["smooth_v"], return_lse=c["lse"], kernel=kern, **kw)
        torch.cuda.synchronize()
        outs[kern] = tuple(t.cpu() for t in r) if c["lse"] else (r.cpu(),)
    for kern in kernels[1:]:
        if kern == 4:
            check(outs[4][0], outs[4][1] if c["lse"] else None)
            continue
        for a, b in zip(outs[1], outs[kern]):
            assert torch.equal(a, b), (kern, (a.float() - b.float()).abs().max().item())
    chosen = lib.kernel_choice(c["B"], c["H"], c["N"], c["D"], c["causal"])
    assert torch.equal(outs[chosen][0], out), chosen
    if c["lse"]:
        assert torch.equal(outs[chosen][1], lse.cpu()), chosen
