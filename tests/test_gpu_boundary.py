"""The library's boundary entries beyond the packed-constant main loop (GPU tests).

* `sage_attn_fwd_sk` runs the main loop on the reference kernel's own inputs (K8, SK, V8T, SV', S
  as the reference prologue leaves them). Fed the ORACLE's quantized tensors, it must give the same
  output, logsumexp rows and smooth_v output bits as the library's packed-constant path fed its own
  prologue (whose tensors equal the oracle's bit for bit, checked in the quantizer tests).
* `sage_kseq_mean` (`HipPrologue.kseq_mean`) is the oracle's fp64 mean, bit for bit.
* `HipPrologue.quant_kv` (the reference's prologue interface) gives the oracle's tensors.
* Grids are 1-D over (plane, block): B*H beyond 65535 is served, and each plane's output is the one
  it has when computed on its own.
"""
import pytest
import torch

import oracle
from sage_testutil import (bytes_equal, cosine, have_gfx950, make_qkv, mismatch_report, rel_l1,
                           rel_l1_bar)

pytestmark = [pytest.mark.gpu,
              pytest.mark.skipif(not have_gfx950(), reason="needs a gfx950 GPU")]

PIPE = 3


def _lib():
    from sageattention.sk1_backend.sk1_loader import SageLib
    return SageLib.get()


def _oracle_kv(k, v, *, k_int8, smooth_k, smooth_v):
    B, H_kv, N_kv, D = k.shape
    kr, vr = k.reshape(B * H_kv, N_kv, D), v.reshape(B * H_kv, N_kv, D)
    n_pad = oracle.n_pad_for(N_kv)
    mean = oracle.kseq_mean(kr) if smooth_k else None
    vmean = oracle.kseq_mean(vr) if smooth_v else None
    k8, sk = oracle.quant_k(kr, n_pad, mean=mean, int8=k_int8)
    v8t, sv = oracle.quant_v(vr, n_pad, mean=vmean)
    s, svp = oracle.fold_v_scale(sv)
    return dict(mean=mean, vmean=vmean, k8=k8, sk=sk, v8t=v8t, svp=svp, s=s)


SK_CASES = [
    # (dtype, B, H, H_kv, N, N_kv, causal, D)
    (torch.float16, 1, 2, 2, 1, 1, False, 128),
    (torch.float16, 1, 3, 3, 300, 300, True, 128),
    (torch.float16, 2, 2, 2, 1337, 1337, False, 128),
    (torch.bfloat16, 1, 2, 2, 700, 700, True, 128),
    (torch.bfloat16, 2, 2, 2, 129, 129, False, 128),
    (torch.float16, 1, 4, 2, 513, 513, True, 128),
    (torch.float16, 1, 4, 4, 70, 1000, False, 128),
    (torch.bfloat16, 1, 8, 2, 1000, 77, False, 128),
    (torch.float16, 1, 3, 3, 257, 257, True, 64),
    (torch.bfloat16, 2, 2, 1, 300, 300, False, 64),
]


@pytest.mark.parametrize("smooth", ["none", "k", "kv"])
@pytest.mark.parametrize("case", SK_CASES, ids=lambda c: "%s-B%dH%dkv%dN%dNk%d%s-D%d" % (
    str(c[0]).split(".")[-1], c[1], c[2], c[3], c[4], c[5], "c" if c[6] else "", c[7]))
def test_main_loop_on_oracle_sk_svp_is_bitwise_the_packed_path(case, smooth):
    from sageattention.sk1_backend import sk1_forward
    dtype, B, H, H_kv, N, N_kv, causal, D = case
    smooth_k, smooth_v = smooth in ("k", "kv"), smooth == "kv"
    print("sk entry", case, smooth, flush=True)
    q, k, v = make_qkv(B, H, N, seed=N + 7 * N_kv + D, dtype=dtype, k_offset_std=2.0,
                       outlier_frac=0.01, d=D, h_kv=H_kv, n_kv=N_kv, v_offset_std=1.0)
    v[0, 0, N_kv // 2] = 3000.0 if dtype == torch.float16 else 6000.0   # S > 1 on one plane
    qk_int8 = dtype == torch.float16
    ref = _oracle_kv(k, v, k_int8=qk_int8, smooth_k=smooth_k, smooth_v=smooth_v)
    lib = _lib()
    sm = D ** -0.5
    o_ref, lse_ref = sk1_forward(lib, q.cuda(), k.cuda(), v.cuda(), is_causal=causal,
                                 smooth_k=smooth_k, smooth_v=smooth_v, kernel=PIPE,
                                 return_lse=True)
    qd = q.cuda()
    o = torch.full_like(qd, float("nan"))
    lse = torch.full((B, H, N), float("nan"), device="cuda")
    dev = lambda t: None if t is None else t.cuda()  # noqa: E731
    lib.attn_fwd_sk(qd, dev(ref["k8"]), dev(ref["sk"]), dev(ref["v8t"]), dev(ref["svp"]),
                    dev(ref["s"]), o, qk_int8=qk_int8, causal=causal, sm_scale=sm, n_kv=N_kv,
                    vmean=dev(ref["vmean"]), lse=lse, kmean=dev(ref["mean"]))
    torch.cuda.synchronize()
    assert torch.equal(o.cpu(), o_ref.cpu()), mismatch_report(o.cpu(), o_ref.cpu(), "o")
    assert torch.equal(lse.cpu(), lse_ref.cpu()), mismatch_report(lse.cpu(), lse_ref.cpu(), "lse")


def test_main_loop_on_sk_svp_matches_emulation():
    q, k, v = make_qkv(2, 2, 1337, seed=5, dtype=torch.float16, k_offset_std=2.0,
                       outlier_frac=0.001)
    ref = _oracle_kv(k, v, k_int8=True, smooth_k=True, smooth_v=False)
    em = oracle.emulate_sageattn(q, k, v, tensor_layout="HND", is_causal=True)["o"]
    qd = q.cuda()
    o = torch.empty_like(qd)
    _lib().attn_fwd_sk(qd, ref["k8"].cuda(), ref["sk"].cuda(), ref["v8t"].cuda(),
                       ref["svp"].cuda(), ref["s"].cuda(), o, qk_int8=True, causal=True,
                       sm_scale=128 ** -0.5)
    torch.cuda.synchronize()
    assert cosine(o.cpu(), em) >= 0.999 and rel_l1(o.cpu(), em) <= rel_l1_bar(True)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("N,D,layout", [(1, 128, "HND"), (63, 128, "HND"), (5000, 128, "NHD"),
                                        (47520, 128, "HND"), (777, 64, "HND")])
def test_kseq_mean_entry_bit_exact(dtype, N, D, layout):
    from sageattention.sk1_backend.hip_prologue import HipPrologue
    H = 3 if N < 40000 else 1
    _, k, _ = make_qkv(2, H, N, seed=N + D, dtype=dtype, k_offset_std=2.0, d=D, layout=layout)
    kk = oracle.to_hnd(k, layout)
    ref = oracle.kseq_mean(kk.reshape(-1, N, D)).view(2, H, D)
    got = HipPrologue(_lib()).kseq_mean(oracle.to_hnd(k.cuda(), layout))
    assert got is not None
    torch.cuda.synchronize()
    assert bytes_equal(got.cpu(), ref), mismatch_report(got.cpu(), ref, "mean")


@pytest.mark.parametrize("dtype,int8", [(torch.float16, True), (torch.float16, False),
                                        (torch.bfloat16, False)])
def test_hip_prologue_quant_kv_bit_exact(dtype, int8):
    from sageattention.sk1_backend.hip_prologue import HipPrologue
    _, k, v = make_qkv(2, 3, 1000, seed=17, dtype=dtype, k_offset_std=2.0, outlier_frac=0.001)
    v[1, 2, 5] = 5000.0
    ref = _oracle_kv(k, v, k_int8=int8, smooth_k=True, smooth_v=False)
    hp = HipPrologue(_lib())
    got = hp.quant_kv(k.cuda(), v.cuda(), smooth_k=True, int8=int8, fold=True, mean_out=True)
    assert got is not None, hp.refusal_reasons
    torch.cuda.synchronize()
    k8, sk, v8t, svp, s, mean = (t.cpu() for t in got)
    for name, a, b in (("k8", k8, ref["k8"]), ("sk", sk, ref["sk"]), ("v8t", v8t, ref["v8t"]),
                       ("svp", svp, ref["svp"]), ("s", s, ref["s"]), ("mean", mean, ref["mean"])):
        assert bytes_equal(a, b), mismatch_report(a, b, name)
    # refusals return None and are counted (the reference's "never raises" contract)
    other = torch.bfloat16 if dtype == torch.float16 else torch.float16
    refused = hp.quant_kv(k.cuda(), v.cuda().to(other), int8=int8) is None
    assert refused and hp.refusal_reasons["dtype_mismatch"] == 1


def test_more_planes_than_a_grid_dimension():
    # B*H = 70,000 planes (beyond 65535): every kernel's grid is 1-D over (plane, block), so
    # each plane's output must be the one it has when computed alone, and match the emulation
    from sageattention import sageattn
    B, H, N, D = 1, 70000, 40, 64
    g = torch.Generator().manual_seed(70000)
    q = torch.randn(B, H, N, D, generator=g).to(torch.float16)
    k = (torch.randn(B, H, N, D, generator=g) + 1.5).to(torch.float16)
    v = torch.randn(B, H, N, D, generator=g).to(torch.float16)
    print("B*H = 70000 N 40 D 64", flush=True)
    for causal in (False, True):
        out = sageattn(q.cuda(), k.cuda(), v.cuda(), tensor_layout="HND", is_causal=causal)
        torch.cuda.synchronize()
        out = out.cpu()
        pick = [0, 1, 32767, 65535, 65536, 69998, 69999]
        qs, ks, vs = (t[:, pick].contiguous() for t in (q, k, v))
        alone = sageattn(qs.cuda(), ks.cuda(), vs.cuda(), tensor_layout="HND",
                         is_causal=causal).cpu()
        assert torch.equal(out[:, pick], alone)
        em = oracle.emulate_sageattn(qs, ks, vs, tensor_layout="HND", is_causal=causal)["o"]
        assert cosine(alone, em) >= 0.999 and rel_l1(alone, em) <= rel_l1_bar(True)
        assert torch.isfinite(out).all()


def test_loaded_library_is_built_from_this_tree():
    # on the GPU box the library is loaded as built here: its build id must be this tree's
    import build_lib
    assert _lib().build_id == build_lib.source_hash()
