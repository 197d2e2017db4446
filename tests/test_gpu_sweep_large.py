"""A seeded sweep of large call shapes through the served path (GPU): the grids where the
automatic kernel choice runs the 256-query ping-pong or the pipelined kernel at many blocks per CU.

Each case draws batch, heads, K/V heads (GQA/MQA), query length 2048..16384, key length, head_dim,
dtype, layout, causality, smooth_k, smooth_v and return_lse, then checks:
* three 64-row slices of the output (first, middle, last query rows) against the CPU emulation of
  just those rows (`sage_testutil.emulate_rows`, pinned against the full emulation on the CPU):
  cosine >= 0.999, rel-L1 <= 1e-2; with return_lse, those rows' logsumexp within the bound of
  tests/test_gpu_sweep.py;
* every main-loop kernel that serves the shape with the served call's arithmetic bit for bit
  against the served call, and the others (the key split or kernels 1-3, whichever was not
  chosen) on the same rows against the emulation.
"""
import random

import pytest
import torch

import oracle
from sage_testutil import cosine, emulate_rows, have_gfx950, make_qkv, rel_l1, rel_l1_bar

pytestmark = [pytest.mark.gpu,
              pytest.mark.skipif(not have_gfx950(), reason="needs a gfx950 GPU")]

N_CASES = 48


def _draw(seed):
    r = random.Random(seed)
    D = r.choice([64, 128, 128])
    dtype = r.choice([torch.float16, torch.float16, torch.bfloat16])
    causal = r.random() < 0.5
    N = r.choice([2048, 3000, 4096, 6144, 8192, 12000, 16384])
    N_kv = N if causal else r.choice([N, 4096, 9000])
    H_kv = r.choice([1, 2, 4, 8])
    H = H_kv * r.choice([1, 2, 4])
    B = r.choice([1, 2])
    while B * H * max(N, N_kv) > (1 << 19):      # bounds the CPU side (inputs and prologue)
        if B > 1:
            B -= 1
        else:
            H, H_kv = max(1, H // 2), max(1, H_kv // 2)
    return dict(D=D, dtype=dtype, causal=causal, B=B, H=H, H_kv=H_kv, N=N, N_kv=N_kv,
                layout=r.choice(["HND", "NHD"]), smooth_k=r.random() < 0.8,
                smooth_v=r.random() < 0.3, lse=r.random() < 0.4)


@pytest.mark.parametrize("seed", range(N_CASES))
def test_large_shape(seed):
    from sageattention import sageattn
    from sageattention.sk1_backend import sk1_forward
    from sageattention.sk1_backend.sk1_loader import SageLib
    c = _draw(5000 + seed)
    print("case", seed, c, flush=True)
    q, k, v = make_qkv(c["B"], c["H"], c["N"], seed=seed, dtype=c["dtype"], layout=c["layout"],
                       k_offset_std=2.0, outlier_frac=1e-3, d=c["D"], h_kv=c["H_kv"],
                       n_kv=c["N_kv"], v_offset_std=1.0 if c["smooth_v"] else 0.0)
    kw = dict(tensor_layout=c["layout"], is_causal=c["causal"])
    res = sageattn(q.cuda(), k.cuda(), v.cuda(), return_lse=c["lse"], smooth_k=c["smooth_k"],
                   smooth_v=c["smooth_v"], **kw)
    torch.cuda.synchronize()
    out, lse = (res if c["lse"] else (res, None))
    out = out.cpu()
    assert torch.isfinite(out).all()
    out_hnd = oracle.to_hnd(out, c["layout"])
    N = c["N"]
    slices = (range(0, 64), range(N // 2 - 32, N // 2 + 32), range(N - 64, N))
    got, ref, got_lse, ref_lse = [], [], [], []
    for rows in slices:
        o_r, lse_r = emulate_rows(q, k, v, rows, smooth_k=c["smooth_k"], smooth_v=c["smooth_v"],
                                  **kw)
        got.append(out_hnd[:, :, rows.start:rows.stop])
        ref.append(o_r)
        if c["lse"]:
            got_lse.append(lse.cpu()[:, :, rows.start:rows.stop])
            ref_lse.append(lse_r)
    got, ref = torch.cat(got, dim=2), torch.cat(ref, dim=2)
    cs, rl = cosine(got, ref), rel_l1(got, ref)
    assert cs >= 0.999 and rl <= rel_l1_bar(c["dtype"] == torch.float16), (cs, rl)
    if c["lse"]:
        g = torch.cat(got_lse, dim=2).double()
        e = torch.cat(ref_lse, dim=2).double()
        # the emulation's logsumexp up to 1e-3 + 1e-4 |lse|, plus the fp8 Q.K score error bound
        # of tests/test_gpu_attention.py when Q.K is fp8 (bf16 inputs)
        tol = 1e-3 + 1e-4 * e.abs()
        if c["dtype"] == torch.bfloat16:
            qq = oracle.to_hnd(q, c["layout"])
            B, H, _, D = qq.shape
            kk = oracle.to_hnd(k, c["layout"]).reshape(B * c["H_kv"], c["N_kv"], D)
            mean = oracle.kseq_mean(kk) if c["smooth_k"] else None
            _, sk = oracle.quant_k(kk, oracle.n_pad_for(c["N_kv"]), mean=mean, int8=False)
            rows_q = torch.cat([qq[:, :, r.start:r.stop] for r in slices], dim=2)
            _, _, cq = oracle.quant_q(rows_q.reshape(B * H, -1, D), D ** -0.5, int8=False)
            tol = tol + 2.0 ** -10 * 448 ** 2 * cq.view_as(e).double() * sk.amax().item() / float(
                oracle.LOG2E)
        assert ((g - e).abs() <= tol).all(), (g - e).abs().max().item()
    # the kernels 1-3 that serve the shape give the served call's bits when it ran one of them;
    # the key split (non-causal head_dim 64) gives them when it was chosen, and otherwise the
    # same rows within the emulation bound
    lib = SageLib.get()
    chosen = lib.kernel_choice(c["B"], c["H"], c["N"], c["D"], c["causal"])
    kernels = [1, 3] + ([2] if c["D"] == 128 else []) + (
        [4] if c["D"] == 64 and not c["causal"] else [])
    for kern in kernels:
        r = sk1_forward(lib, q.cuda(), k.cuda(), v.cuda(), smooth_k=c["smooth_k"],
                        smooth_v=c["smooth_v"], return_lse=c["lse"], kernel=kern, **kw)
        torch.cuda.synchronize()
        o = (r[0] if c["lse"] else r).cpu()
        if (kern == 4) == (chosen == 4):
            assert torch.equal(o, out), kern
            if c["lse"]:
                assert torch.equal(r[1].cpu(), lse.cpu()), kern
        else:
            o_hnd = oracle.to_hnd(o, c["layout"])
            g = torch.cat([o_hnd[:, :, rows.start:rows.stop] for rows in slices], dim=2)
            cs, rl = cosine(g, ref), rel_l1(g, ref)
            assert cs >= 0.999 and rl <= rel_l1_bar(c["dtype"] == torch.float16), (kern, cs, rl)
