"""The committed golden fixtures (tests/golden/*.npz, written by tests/golden/make_golden.py).

* CPU: the oracle, re-run on each fixture's stored input bits, must reproduce every stored array
  bit for bit (the oracle has not drifted since the fixtures were frozen).
* GPU: the gfx950 library on the same input bits must reproduce every quantized tensor and scale
  bit for bit, and the output of `sageattn` must meet the accuracy bar against the stored emulated
  output (cosine >= 0.999, relative L1 <= 1e-2).
"""
import glob
import os

import numpy as np
import pytest
import torch

import oracle
from sage_testutil import COS_MIN, cosine, have_gfx950, rel_l1, rel_l1_bar

GOLDEN = sorted(glob.glob(os.path.join(os.path.dirname(__file__), "golden", "*.npz")))


def _load(path):
    with np.load(path, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def _inputs(g):
    B, H, N, causal, smooth_k, nhd, bf16, H_kv, N_kv, smooth_v, D = (int(x) for x in g["meta"])
    dtype = torch.bfloat16 if bf16 else torch.float16
    shape = (B, N, H, D) if nhd else (B, H, N, D)
    kv_shape = (B, N_kv, H_kv, D) if nhd else (B, H_kv, N_kv, D)
    q = torch.from_numpy(g["q"].astype(np.int16)).view(dtype).reshape(shape)
    k, v = (torch.from_numpy(g[n].astype(np.int16)).view(dtype).reshape(kv_shape) for n in "kv")
    return q, k, v, dict(causal=bool(causal), smooth_k=bool(smooth_k), smooth_v=bool(smooth_v),
                         layout="NHD" if nhd else "HND", dtype=dtype)


def _bits(t):
    t = t.contiguous()
    if t.dtype in (torch.float16, torch.bfloat16):
        return t.view(torch.int16).numpy().view(np.uint16)
    if t.dtype == torch.float8_e4m3fn:
        return t.view(torch.uint8).numpy()
    return t.numpy()


def test_fixtures_present():
    assert len(GOLDEN) >= 4, GOLDEN


@pytest.mark.parametrize("path", GOLDEN, ids=lambda p: os.path.basename(p)[:-4])
def test_oracle_reproduces_fixture(path):
    g = _load(path)
    q, k, v, m = _inputs(g)
    r = oracle.emulate_sageattn(q, k, v, tensor_layout=m["layout"], is_causal=m["causal"],
                                smooth_k=m["smooth_k"], smooth_v=m["smooth_v"])
    for name in ("k8", "sk", "v8t", "sv", "s", "svp", "q8", "sq", "c_q", "o", "lse"):
        assert np.array_equal(_bits(r[name]), g[name]), name
    if m["smooth_k"]:
        assert np.array_equal(r["mean"].numpy(), g["mean"])
    if m["smooth_v"]:
        assert np.array_equal(r["vmean"].numpy(), g["vmean"])
    assert np.float32(r["sm_scale"]) == g["sm_scale"][0]


@pytest.mark.gpu
@pytest.mark.skipif(not have_gfx950(), reason="needs a gfx950 GPU")
@pytest.mark.parametrize("path", GOLDEN, ids=lambda p: os.path.basename(p)[:-4])
def test_gpu_matches_fixture(path):
    from sageattention import sageattn
    from sageattention.sk1_backend.sk1_loader import SageLib
    g = _load(path)
    q, k, v, m = _inputs(g)
    print("fixture", os.path.basename(path), tuple(q.shape), m, flush=True)
    lib = SageLib.get()
    qd, kd, vd = (t.cuda() for t in (q, k, v))
    kk, vv, qq = (oracle.to_hnd(t, m["layout"]) for t in (kd, vd, qd))
    B, H, N, D = kk.shape
    BH, n_pad = B * H, oracle.n_pad_for(N)
    int8 = m["dtype"] == torch.float16
    dev = qd.device
    k8 = torch.empty(BH, n_pad, D, device=dev, dtype=torch.int8 if int8 else torch.float8_e4m3fn)
    v8t = torch.empty(BH, D, n_pad, device=dev, dtype=torch.float8_e4m3fn)
    sk, sv = (torch.empty(BH, n_pad, device=dev) for _ in range(2))
    s, mean = torch.empty(BH, device=dev), torch.empty(BH, D, device=dev)
    vmean = torch.empty(BH, D, device=dev)
    ws = torch.empty(lib.workspace_bytes(BH, N), device=dev, dtype=torch.uint8)
    lib.kv_prologue(kk, vv, k8, sk, v8t, sv, s, mean, ws, k_int8=int8, smooth_k=m["smooth_k"],
                    fold=True, n_pad=n_pad, smooth_v=m["smooth_v"], vmean=vmean)
    q8, sq, cq = lib.quant_q(qq, float(g["sm_scale"][0]), qk_int8=int8)
    out, lse = sageattn(qd, kd, vd, tensor_layout=m["layout"], is_causal=m["causal"],
                        smooth_k=m["smooth_k"], smooth_v=m["smooth_v"], return_lse=True)
    torch.cuda.synchronize()
    got = dict(k8=k8, v8t=v8t, sk=sk, svp=sv, s=s, q8=q8, sq=sq, c_q=cq)
    for name, t in got.items():
        assert np.array_equal(_bits(t.cpu()), g[name]), name
    if m["smooth_k"]:
        assert np.array_equal(mean.cpu().numpy(), g["mean"])
    if m["smooth_v"]:
        assert np.array_equal(vmean.cpu().numpy(), g["vmean"])
    ref = torch.from_numpy(g["o"].astype(np.int16)).view(m["dtype"]).reshape(out.shape)
    c, r1 = cosine(out.cpu(), ref), rel_l1(out.cpu(), ref)
    print("cos %.6f rel_l1 %.3e" % (c, r1), flush=True)
    assert c >= COS_MIN and r1 <= rel_l1_bar(int8)
    # logsumexp: same quantized scores, hardware exp2/log2 and another summation order
    lref = torch.from_numpy(g["lse"])
    assert lse.shape == lref.shape and lse.dtype == torch.float32
    assert torch.allclose(lse.cpu(), lref, rtol=1e-4, atol=1e-3), (lse.cpu() - lref).abs().max()
