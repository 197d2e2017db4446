"""Bit-exact parity of the gfx950 quantizers with the CPU oracle (GPU tests).

Every quantized tensor and scale of the scheme -- mu, K8, SK, V8T, SV, S, SV', Q8, sq, c_q -- must
equal the oracle's bits. Outputs are prefilled with sentinels first, so a pad row the kernels fail
to write shows up as a mismatch.
"""
import pytest
import torch

import oracle
from sage_testutil import HEAD_DIM, bytes_equal, have_gfx950, make_qkv, mismatch_report

pytestmark = [pytest.mark.gpu,
              pytest.mark.skipif(not have_gfx950(), reason="needs a gfx950 GPU")]


def _lib():
    from sageattention.sk1_backend.sk1_loader import SageLib
    return SageLib.get()


def _run_prologue(k, v, *, k_int8, smooth_k, fold, layout="HND", with_kconst=False,
                  smooth_v=False):
    lib = _lib()
    kk, vv = (oracle.to_hnd(t, layout) for t in (k, v))
    B, H, N, D = kk.shape
    BH = B * H
    n_pad = oracle.n_pad_for(N)
    dev = k.device
    k8 = torch.full((BH, n_pad, D), 0x5A, device=dev, dtype=torch.uint8)
    k8 = k8.view(torch.int8 if k_int8 else torch.float8_e4m3fn)
    v8t = torch.full((BH, D, n_pad), 0x5A, device=dev, dtype=torch.uint8).view(torch.float8_e4m3fn)
    sk = torch.full((BH, n_pad), float("nan"), device=dev)
    sv = torch.full((BH, n_pad), float("nan"), device=dev)
    s = torch.full((BH,), float("nan"), device=dev)
    mean = torch.full((BH, D), float("nan"), device=dev)
    vmean = torch.full((BH, D), float("nan"), device=dev)
    ws = torch.full((lib.workspace_bytes(BH, N),), 0xFF, device=dev, dtype=torch.uint8)
    kc = (torch.full((BH, n_pad // 64, 2, 64), float("nan"), device=dev) if with_kconst
          else None)
    lib.kv_prologue(kk, vv, k8, sk, v8t, sv, s, mean, ws, k_int8=k_int8, smooth_k=smooth_k,
                    fold=fold, n_pad=n_pad, kconst=kc, smooth_v=smooth_v, vmean=vmean)
    torch.cuda.synchronize()
    out = dict(k8=k8.cpu(), sk=sk.cpu(), v8t=v8t.cpu(), sv=sv.cpu(), s=s.cpu(), mean=mean.cpu(),
               vmean=vmean.cpu())
    if with_kconst:
        out["kconst"] = kc.cpu()
    return out


def _oracle_prologue(k, v, *, k_int8, smooth_k, layout="HND", smooth_v=False):
    kk, vv = (oracle.to_hnd(t, layout) for t in (k, v))
    B, H, N, D = kk.shape
    kr, vr = kk.reshape(B * H, N, D), vv.reshape(B * H, N, D)
    n_pad = oracle.n_pad_for(N)
    mean = oracle.kseq_mean(kr) if smooth_k else None
    vmean = oracle.kseq_mean(vr) if smooth_v else None
    k8, sk = oracle.quant_k(kr, n_pad, mean=mean, int8=k_int8)
    v8t, sv = oracle.quant_v(vr, n_pad, mean=vmean)
    s, svp = oracle.fold_v_scale(sv)
    return dict(mean=mean, vmean=vmean, k8=k8, sk=sk, v8t=v8t, sv=sv, s=s, svp=svp)


CASES = [
    # (dtype, k_int8, N, H, k_offset, outliers, std)
    (torch.float16, True, 1, 2, 2.0, 0.0, 1.0),
    (torch.float16, True, 63, 2, 2.0, 0.0, 1.0),
    (torch.float16, True, 64, 3, 2.0, 0.0, 1.0),
    (torch.float16, True, 65, 2, 2.0, 0.0, 1.0),
    (torch.float16, True, 300, 2, 2.0, 0.01, 1.0),
    (torch.float16, True, 1000, 4, 2.0, 0.001, 1.0),
    (torch.float16, True, 8771, 2, 2.0, 0.001, 1.0),
    (torch.float16, False, 300, 2, 2.0, 0.0, 1.0),
    (torch.bfloat16, False, 1, 2, 2.0, 0.0, 1.5),
    (torch.bfloat16, False, 129, 2, 2.0, 0.0, 1.5),
    (torch.bfloat16, False, 1000, 3, 2.0, 0.001, 1.5),
    (torch.bfloat16, False, 16384, 1, 2.0, 0.001, 1.5),
]


@pytest.mark.parametrize("smooth_k", [True, False])
@pytest.mark.parametrize("case", CASES, ids=lambda c: "%s-%s-N%d" % (
    str(c[0]).split(".")[-1], "i8" if c[1] else "f8", c[2]))
def test_prologue_bit_exact(case, smooth_k):
    dtype, k_int8, N, H, off, outl, std = case
    q, k, v = make_qkv(1, H, N, seed=N + H, dtype=dtype, std=std, k_offset_std=off,
                       outlier_frac=outl)
    print("case", case, "smooth_k", smooth_k, flush=True)
    ref = _oracle_prologue(k, v, k_int8=k_int8, smooth_k=smooth_k)
    got = _run_prologue(k.cuda(), v.cuda(), k_int8=k_int8, smooth_k=smooth_k, fold=False)
    if smooth_k:
        assert bytes_equal(got["mean"], ref["mean"]), mismatch_report(got["mean"], ref["mean"], "mean")
    for name in ("k8", "sk", "v8t", "sv", "s"):
        assert bytes_equal(got[name], ref[name]), mismatch_report(got[name], ref[name], name)
    folded = _run_prologue(k.cuda(), v.cuda(), k_int8=k_int8, smooth_k=smooth_k, fold=True)
    assert bytes_equal(folded["sv"], ref["svp"]), mismatch_report(folded["sv"], ref["svp"], "svp")
    assert bytes_equal(folded["k8"], ref["k8"])


@pytest.mark.parametrize("smooth_k", [True, False])
@pytest.mark.parametrize("case", [CASES[0], CASES[2], CASES[3], CASES[4], CASES[6], CASES[8],
                                  CASES[10], CASES[11]], ids=lambda c: "%s-%s-N%d" % (
    str(c[0]).split(".")[-1], "i8" if c[1] else "f8", c[2]))
def test_prologue_smooth_v_bit_exact(case, smooth_k):
    # smooth_v: V's fp64 sequence mean, V centred before its per-token scale (a second stats
    # launch); K's outputs must not move; S > 1 (a V row far above 448) exercises the fold.
    dtype, k_int8, N, H, off, outl, std = case
    q, k, v = make_qkv(1, H, N, seed=N + 2 * H, dtype=dtype, std=std, k_offset_std=off,
                       outlier_frac=outl, v_offset_std=3.0)
    if N > 5:
        v[0, 0, 5] = 3000.0
    print("case", case, "smooth_k", smooth_k, flush=True)
    ref = _oracle_prologue(k, v, k_int8=k_int8, smooth_k=smooth_k, smooth_v=True)
    got = _run_prologue(k.cuda(), v.cuda(), k_int8=k_int8, smooth_k=smooth_k, fold=True,
                        smooth_v=True)
    assert bytes_equal(got["vmean"], ref["vmean"]), mismatch_report(got["vmean"], ref["vmean"],
                                                                    "vmean")
    if smooth_k:
        assert bytes_equal(got["mean"], ref["mean"]), mismatch_report(got["mean"], ref["mean"], "mean")
    for name, rname in (("k8", "k8"), ("sk", "sk"), ("v8t", "v8t"), ("sv", "svp"), ("s", "s")):
        assert bytes_equal(got[name], ref[rname]), mismatch_report(got[name], ref[rname], name)
    plain = _run_prologue(k.cuda(), v.cuda(), k_int8=k_int8, smooth_k=smooth_k, fold=True)
    assert bytes_equal(plain["k8"], got["k8"]) and bytes_equal(plain["sk"], got["sk"])


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_prologue_v_outlier_fold(dtype):
    # |V| far above 448 makes S > 1, so SV' = SV / S differs from SV (the reference's outlier case).
    q, k, v = make_qkv(1, 2, 1024, seed=1, dtype=dtype)
    v[:, :, 300] = 20000.0
    k_int8 = dtype == torch.float16
    ref = _oracle_prologue(k, v, k_int8=k_int8, smooth_k=True)
    assert (ref["s"] > 1).all()
    got = _run_prologue(k.cuda(), v.cuda(), k_int8=k_int8, smooth_k=True, fold=True)
    for name, rname in (("k8", "k8"), ("sk", "sk"), ("v8t", "v8t"), ("sv", "svp"), ("s", "s")):
        assert bytes_equal(got[name], ref[rname]), mismatch_report(got[name], ref[rname], name)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_prologue_strided_views_same_bits(dtype):
    # NHD input read through strides gives the same bytes as contiguous HND.
    q, k, v = make_qkv(2, 4, 300, seed=3, dtype=dtype, k_offset_std=2.0)
    k_int8 = dtype == torch.float16
    a = _run_prologue(k.cuda(), v.cuda(), k_int8=k_int8, smooth_k=True, fold=True)
    kn, vn = (t.transpose(1, 2).contiguous().cuda() for t in (k, v))
    b = _run_prologue(kn, vn, k_int8=k_int8, smooth_k=True, fold=True, layout="NHD")
    for name in ("k8", "sk", "v8t", "sv", "s", "mean"):
        assert bytes_equal(a[name], b[name]), name


@pytest.mark.parametrize("case", [CASES[3], CASES[4], CASES[9], CASES[10]], ids=lambda c: "%s-%s-N%d" % (
    str(c[0]).split(".")[-1], "i8" if c[1] else "f8", c[2]))
def test_prologue_kconst_layout(case):
    # The main loop's per-key constants: for each 64-key block, SK and RN(SV'*448), the second one
    # fp32 rounding of the prologue's own SV' bits.
    dtype, k_int8, N, H, off, outl, std = case
    q, k, v = make_qkv(1, H, N, seed=N + 7, dtype=dtype, std=std, k_offset_std=off,
                       outlier_frac=outl)
    v[0, 0, 0, :4] = 1000.0                 # S > 1: the constants must use the folded SV'
    print("case", case, flush=True)
    got = _run_prologue(k.cuda(), v.cuda(), k_int8=k_int8, smooth_k=True, fold=True,
                        with_kconst=True)
    BH, n_pad = H, oracle.n_pad_for(N)
    kc = got["kconst"].reshape(BH, n_pad // 64, 2, 64)
    sk = got["sk"].reshape(BH, n_pad // 64, 64)
    svp = got["sv"].reshape(BH, n_pad // 64, 64)
    want_w = svp * oracle.P_SCALE
    assert bytes_equal(kc[:, :, 0].contiguous(), sk), mismatch_report(kc[:, :, 0], sk, "kc.sk")
    assert bytes_equal(kc[:, :, 1].contiguous(), want_w), mismatch_report(kc[:, :, 1], want_w, "kc.w")
    ref = _oracle_prologue(k, v, k_int8=k_int8, smooth_k=True)
    assert bytes_equal(got["sv"], ref["svp"])


@pytest.mark.parametrize("dtype,qk_int8", [(torch.float16, True), (torch.float16, False),
                                           (torch.bfloat16, False)])
@pytest.mark.parametrize("N", [1, 31, 33, 300, 4097])
def test_quant_q_bit_exact(dtype, qk_int8, N):
    q, k, v = make_qkv(1, 3, N, seed=7 + N, dtype=dtype, std=1.5)
    q[0, 1, : min(N, 5)] = 0.0          # all-zero rows take the 1e-12 floor
    if N > 10:
        q[0, 2, 7, 3] = 60000.0 if dtype == torch.float16 else 3.0e5   # a huge element
    sm = HEAD_DIM ** -0.5
    q8, sq, cq = _lib().quant_q(q.cuda(), sm, qk_int8=qk_int8)
    torch.cuda.synchronize()
    r8, rsq, rcq = oracle.quant_q(q.reshape(3, N, HEAD_DIM), sm, int8=qk_int8)
    assert bytes_equal(q8.cpu(), r8), mismatch_report(q8.cpu(), r8, "q8")
    assert bytes_equal(sq.cpu(), rsq), mismatch_report(sq.cpu(), rsq, "sq")
    assert bytes_equal(cq.cpu(), rcq), mismatch_report(cq.cpu(), rcq, "cq")


def test_fp8_convert_matches_torch_on_all_fp16_in_range():
    # Every finite fp16 value with |x| <= 448 quantized as a V row with sv = 1: e4m3(min(x/1, 448))
    # must equal torch's float8_e4m3fn cast, i.e. the hardware convert is OCP e4m3fn with RNE.
    allv = torch.arange(0, 1 << 16, dtype=torch.int32).to(torch.int16).view(torch.float16)
    vals = allv[torch.isfinite(allv) & (allv.float().abs() <= 448)]
    n = vals.numel() // HEAD_DIM * HEAD_DIM
    vals = vals[:n].reshape(1, 1, n // HEAD_DIM, HEAD_DIM).clone()
    vals[..., 0] = 448.0                  # every row's absmax is 448, so sv == 1 exactly
    k = torch.zeros_like(vals)
    got = _run_prologue(k.cuda(), vals.cuda(), k_int8=True, smooth_k=False, fold=False)
    rows = vals.shape[2]
    ref = vals.reshape(rows, HEAD_DIM).float().to(torch.float8_e4m3fn).t()
    assert (got["sv"][0, :rows] == 1.0).all()
    assert bytes_equal(got["v8t"][0, :, :rows].contiguous(), ref.contiguous())


D64_CASES = [
    # (dtype, k_int8, N, H, k_offset, outliers, std)
    (torch.float16, True, 1, 2, 2.0, 0.0, 1.0),
    (torch.float16, True, 65, 2, 2.0, 0.0, 1.0),
    (torch.float16, True, 300, 3, 2.0, 0.01, 1.0),
    (torch.float16, True, 4097, 2, 2.0, 0.001, 1.0),
    (torch.float16, False, 300, 2, 2.0, 0.0, 1.0),
    (torch.bfloat16, False, 129, 2, 2.0, 0.0, 1.5),
    (torch.bfloat16, False, 2000, 3, 2.0, 0.001, 1.5),
]


@pytest.mark.parametrize("smooth_v", [False, True])
@pytest.mark.parametrize("smooth_k", [True, False])
@pytest.mark.parametrize("case", D64_CASES, ids=lambda c: "%s-%s-N%d" % (
    str(c[0]).split(".")[-1], "i8" if c[1] else "f8", c[2]))
def test_prologue_d64_bit_exact(case, smooth_k, smooth_v):
    # head_dim 64: 8 column groups x 32 row groups, 256-row stats steps (blocks of a multiple of
    # 256 rows), the same arithmetic; a V row far above 448 exercises the fold.
    dtype, k_int8, N, H, off, outl, std = case
    q, k, v = make_qkv(1, H, N, seed=N + 3 * H, dtype=dtype, std=std, k_offset_std=off,
                       outlier_frac=outl, v_offset_std=2.0, d=64)
    if N > 9:
        v[0, 1, 9] = 5000.0
    print("case", case, smooth_k, smooth_v, flush=True)
    ref = _oracle_prologue(k, v, k_int8=k_int8, smooth_k=smooth_k, smooth_v=smooth_v)
    got = _run_prologue(k.cuda(), v.cuda(), k_int8=k_int8, smooth_k=smooth_k, fold=True,
                        smooth_v=smooth_v, with_kconst=True)
    if smooth_k:
        assert bytes_equal(got["mean"], ref["mean"]), mismatch_report(got["mean"], ref["mean"], "mean")
    if smooth_v:
        assert bytes_equal(got["vmean"], ref["vmean"]), mismatch_report(got["vmean"], ref["vmean"],
                                                                        "vmean")
    for name, rname in (("k8", "k8"), ("sk", "sk"), ("v8t", "v8t"), ("sv", "svp"), ("s", "s")):
        assert bytes_equal(got[name], ref[rname]), mismatch_report(got[name], ref[rname], name)
    n_pad = oracle.n_pad_for(N)
    kc = got["kconst"].reshape(H, n_pad // 64, 2, 64)
    assert bytes_equal(kc[:, :, 0].contiguous(), got["sk"].reshape(H, n_pad // 64, 64))
    w = got["sv"].reshape(H, n_pad // 64, 64) * oracle.P_SCALE
    assert bytes_equal(kc[:, :, 1].contiguous(), w)


@pytest.mark.parametrize("dtype,qk_int8", [(torch.float16, True), (torch.float16, False),
                                           (torch.bfloat16, False)])
@pytest.mark.parametrize("N", [1, 33, 300])
def test_quant_q_d64_bit_exact(dtype, qk_int8, N):
    q, k, v = make_qkv(1, 3, N, seed=11 + N, dtype=dtype, std=1.5, d=64)
    q[0, 1, : min(N, 5)] = 0.0
    sm = 64 ** -0.5
    q8, sq, cq = _lib().quant_q(q.cuda(), sm, qk_int8=qk_int8)
    torch.cuda.synchronize()
    r8, rsq, rcq = oracle.quant_q(q.reshape(3, N, 64), sm, int8=qk_int8)
    assert bytes_equal(q8.cpu(), r8), mismatch_report(q8.cpu(), r8, "q8")
    assert bytes_equal(sq.cpu(), rsq) and bytes_equal(cq.cpu(), rcq)


@pytest.mark.parametrize("dtype,k_int8,B,H,N", [
    (torch.float16, True, 20, 40, 70),      # 800 planes: one stats block per plane (768 slots)
    (torch.bfloat16, False, 40, 60, 33),    # 2400 planes: one quant block per plane too (2048)
    (torch.float16, True, 1, 1, 5000),      # one plane over 40 stats / 79 quant blocks
], ids=["BH800", "BH2400", "BH1-N5000"])
def test_prologue_grid_regimes(dtype, k_int8, B, H, N):
    # The prologue's grids are sized to one round of resident blocks: c = slots / planes blocks per
    # plane, at least one. Each regime must give the oracle's bits (and fill every pad row).
    q, k, v = make_qkv(B, H, N, seed=B * H + N, dtype=dtype, k_offset_std=2.0)
    v[0, 0, N // 2] = 3000.0                 # S > 1 on one plane
    print("grid regime", B, H, N, flush=True)
    ref = _oracle_prologue(k, v, k_int8=k_int8, smooth_k=True)
    got = _run_prologue(k.cuda(), v.cuda(), k_int8=k_int8, smooth_k=True, fold=True)
    assert bytes_equal(got["mean"], ref["mean"]), mismatch_report(got["mean"], ref["mean"], "mean")
    for name, rname in (("k8", "k8"), ("sk", "sk"), ("v8t", "v8t"), ("sv", "svp"), ("s", "s")):
        assert bytes_equal(got[name], ref[rname]), mismatch_report(got[name], ref[rname], name)


@pytest.mark.parametrize("extra", [256, 1024])
@pytest.mark.parametrize("dtype,k_int8", [(torch.float16, True), (torch.bfloat16, False)])
def test_prologue_with_padding_beyond_the_last_block(dtype, k_int8, extra):
    # N_pad may exceed ceil(N/64)*64 (the contract asks only for a multiple of 64 >= N): the
    # stats pass's last block then covers every pad row. K8, SK, V8T, SV', S and the mean must
    # equal the oracle's tensors padded to that length (pad rows: K8 0, SK 1.0, V8T 0, SV' 0),
    # KCONST must hold SK and RN(SV'*448) of every block, and the main loop on these tensors must
    # give the bits of the same call with the normal padding (the extra keys are masked: p = 0).
    lib = _lib()
    N, H = 300, 2
    q, k, v = make_qkv(1, H, N, seed=71, dtype=dtype, k_offset_std=2.0, outlier_frac=0.01)
    print("case", dtype, k_int8, extra, flush=True)
    dev = torch.device("cuda:0")
    kd, vd, qd = k.to(dev), v.to(dev), q.to(dev)
    outs = {}
    for n_pad in (oracle.n_pad_for(N), oracle.n_pad_for(N) + extra):
        BH, D = H, HEAD_DIM
        k8 = torch.full((BH, n_pad, D), 0x5A, device=dev, dtype=torch.uint8)
        k8 = k8.view(torch.int8 if k_int8 else torch.float8_e4m3fn)
        v8t = torch.full((BH, D, n_pad), 0x5A, device=dev, dtype=torch.uint8).view(
            torch.float8_e4m3fn)
        sk, sv = (torch.full((BH, n_pad), float("nan"), device=dev) for _ in range(2))
        s = torch.full((BH,), float("nan"), device=dev)
        mean = torch.full((BH, D), float("nan"), device=dev)
        kc = torch.full((BH, n_pad // 64, 2, 64), float("nan"), device=dev)
        ws = torch.full((lib.workspace_bytes(BH, N),), 0xFF, device=dev, dtype=torch.uint8)
        lib.kv_prologue(kd, vd, k8, sk, v8t, sv, s, mean, ws, k_int8=k_int8, smooth_k=True,
                        fold=True, n_pad=n_pad, kconst=kc)
        o = torch.full_like(qd, float("nan"))
        for kernel in (2, 3):
            o.fill_(float("nan"))
            lib.attn_fwd(qd, k8, kc, v8t, s, o, qk_int8=k_int8, causal=False, sm_scale=D ** -0.5,
                         n_pad=n_pad, kernel=kernel)
            torch.cuda.synchronize()
            outs[(n_pad, kernel)] = o.cpu()
        kr, vr = k.reshape(BH, N, D), v.reshape(BH, N, D)
        mu = oracle.kseq_mean(kr)
        r_k8, r_sk = oracle.quant_k(kr, n_pad, mean=mu, int8=k_int8)
        r_v8t, r_sv = oracle.quant_v(vr, n_pad)
        r_s, r_svp = oracle.fold_v_scale(r_sv)
        for got, ref, name in ((mean, mu, "mean"), (k8, r_k8, "k8"), (sk, r_sk, "sk"),
                               (v8t, r_v8t, "v8t"), (sv, r_svp, "svp"), (s, r_s, "s")):
            g = got.cpu()
            assert bytes_equal(g, ref), mismatch_report(g, ref, name)
        kcc = kc.cpu()
        assert bytes_equal(kcc[:, :, 0, :].reshape(BH, n_pad), r_sk)
        assert bytes_equal(kcc[:, :, 1, :].reshape(BH, n_pad), (r_svp * 448.0).float())
    base = oracle.n_pad_for(N)
    for kernel in (2, 3):
        a, b = outs[(base, kernel)], outs[(base + extra, kernel)]
        assert torch.isfinite(b.float()).all()
        assert bytes_equal(a, b), (kernel, mismatch_report(a, b, "o"))
