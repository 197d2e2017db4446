"""Pins of the CPU oracle (CPU tests, no GPU).

The oracle is the checker of every GPU parity test, so it is itself checked against things that do
not share its code: exact rational arithmetic (`exact_ref`), an OCP e4m3 encoder written from the
specification, Python's own half-even rounding, `math.fsum`, brute-force loops on tiny inputs, and
closed forms of attention. A few tests plant a plausible mistake in a copy of an oracle function and
assert that the pin catches it.
"""
import math
import random
from fractions import Fraction

import numpy as np
import pytest
import torch

import oracle
from exact_ref import e4m3_code, e4m3_value, f32_bits, rn32, rne_int
from sage_testutil import make_qkv

F8 = torch.float8_e4m3fn


# ----------------------------------------------------------------------------- n_pad
def test_n_pad_closed_form():
    table = {1: 64, 63: 64, 64: 64, 65: 128, 288: 320, 1024: 1024, 8771: 8832, 16384: 16384,
             47520: 47552}
    for n, p in table.items():
        assert oracle.n_pad_for(n) == p
    for n in range(1, 1000):
        p = oracle.n_pad_for(n)
        assert p % 64 == 0 and p >= n and p - n < 64


# ----------------------------------------------------------------------------- rounding rules
def test_torch_round_is_half_even():
    xs = [0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 126.5, 127.5, -127.5, -128.5, 3.4999998, 0.49999997]
    got = torch.round(torch.tensor(xs, dtype=torch.float32)).tolist()
    assert got == [float(rne_int(Fraction(x))) for x in xs]
    assert got[:6] == [0.0, 2.0, 2.0, -0.0, -2.0, -2.0]


def test_reference_floor_rne_formula_equals_half_even():
    # The reference's int8 K rounding is floor-based (`kernels/hip/h34_prologue.hip:56-64`):
    # fl = floor(x); d = x - fl; q = (d > .5 or (d == .5 and fl odd)) ? fl + 1 : fl, in fp32.
    # Restated with numpy fp32 scalars, it must equal half-even rounding on every fp32 x, including
    # the (-1, 0) range where x - fl is inexact.
    rng = random.Random(0)
    xs = [k / 2 for k in range(-300, 301)]
    xs += [rng.uniform(-130, 130) for _ in range(20000)]
    xs += [float(np.nextafter(np.float32(k / 2), np.float32(s))) for k in range(-260, 261)
           for s in (-1e9, 1e9)]
    xs += [-0.5 + 2.0 ** -25, -0.5 - 2.0 ** -25, -2.0 ** -30, -1 + 2.0 ** -24]
    for x in xs:
        x32 = np.float32(x)
        fl = np.floor(x32)
        d = np.float32(x32 - fl)
        odd = int(fl) & 1
        q = fl + 1 if (d > 0.5 or (d == 0.5 and odd)) else fl
        assert float(q) == float(rne_int(Fraction(float(x32)))), x


# ----------------------------------------------------------------------------- e4m3
def _torch_e4m3_codes(xs):
    return torch.tensor(xs, dtype=torch.float32).to(F8).view(torch.uint8).tolist()


def test_e4m3_cast_matches_ocp_encoder_on_every_fp16_in_range():
    allv = torch.arange(0, 1 << 16, dtype=torch.int32).to(torch.int16).view(torch.float16)
    vals = allv[torch.isfinite(allv) & (allv.float().abs() <= 448)].float()
    got = vals.to(F8).view(torch.uint8).tolist()
    want = [e4m3_code(float(x)) for x in vals.tolist()]
    assert got == want


def test_e4m3_cast_ties_and_boundaries():
    xs, want = [], []
    # every midpoint between consecutive positive codes, and one fp32 ulp either side of it
    for c in range(0, 0x7E):
        lo, hi = e4m3_value(c), e4m3_value(c + 1)
        mid = (lo + hi) / 2
        for x in (float(mid), float(np.nextafter(np.float32(mid), np.float32(0))),
                  float(np.nextafter(np.float32(mid), np.float32(1e9)))):
            xs += [x, -x]
    xs += [448.0, 449.0, 463.99997, 1.0625, 1.1875, 2.0 ** -10, 3 * 2.0 ** -10, 2.0 ** -9]
    want = [e4m3_code(Fraction(x)) for x in xs]
    assert _torch_e4m3_codes(xs) == want
    assert _torch_e4m3_codes([1.0625, 1.1875, 2.0 ** -10, 3 * 2.0 ** -10]) == [0x38, 0x3A, 0x00, 0x02]


# ----------------------------------------------------------------------------- exact pins
def _rn32_div(a, b):
    return rn32(Fraction(a) / Fraction(b))


def _k_int8_exact(row, mu=None):
    """Exact restatement of A.3 for one row: returns (sk, [k8])."""
    kc = [rn32(Fraction(float(x)) - Fraction(float(m))) if mu is not None else float(x)
          for x, m in zip(row, mu if mu is not None else row)]
    kmax = max(abs(x) for x in kc)
    sk = max(_rn32_div(kmax, 127), float(np.float32(1e-12)))
    k8 = [max(-128, min(127, rne_int(_rn32_div(x, sk)))) for x in kc]
    return sk, k8


@pytest.mark.parametrize("d", [128, 64])
def test_quant_k_int8_exact_small(d):
    q, k, v = make_qkv(1, 2, 37, seed=3, k_offset_std=2.0, outlier_frac=0.05, d=d)
    kr = k.reshape(2, 37, d)
    mean = oracle.kseq_mean(kr)
    k8, sk = oracle.quant_k(kr, 64, mean=mean, int8=True)
    for bh in range(2):
        mu = mean[bh].tolist()
        for n in range(37):
            s_ex, q_ex = _k_int8_exact(kr[bh, n].float().tolist(), mu)
            assert f32_bits(sk[bh, n].item()) == f32_bits(s_ex)
            assert k8[bh, n].tolist() == q_ex
        assert (sk[bh, 37:] == 1.0).all() and (k8[bh, 37:] == 0).all()


def test_quant_k_int8_is_a_division_not_a_reciprocal_product():
    # Plant the mistake "kc * RN(1/sk)" in a copy of the quantizer: on these inputs it changes
    # some bytes, so the exact pin above would catch it.
    q, k, v = make_qkv(1, 4, 256, seed=11)
    kr = k.reshape(4, 256, 128)
    k8, sk = oracle.quant_k(kr, 256, int8=True)
    kf = kr.float()
    wrong = torch.clamp(torch.round(kf * (1.0 / sk[:, :, None])), -128, 127).to(torch.int8)
    assert not torch.equal(wrong, k8)
    rows = [(b, n) for b in range(4) for n in range(256) if not torch.equal(wrong[b, n], k8[b, n])]
    b, n = rows[0]
    s_ex, q_ex = _k_int8_exact(kr[b, n].float().tolist())
    assert k8[b, n].tolist() == q_ex and wrong[b, n].tolist() != q_ex


def test_quant_k_fp8_and_v_exact_small():
    q, k, v = make_qkv(1, 1, 20, seed=5, dtype=torch.bfloat16, std=1.5, k_offset_std=2.0)
    kr, vr = k.reshape(1, 20, 128), v.reshape(1, 20, 128)
    k8, sk = oracle.quant_k(kr, 64, int8=False)
    v8t, sv = oracle.quant_v(vr, 64)
    fl = float(np.float32(1e-12))
    for n in range(20):
        row = [float(x) for x in kr[0, n].float().tolist()]
        s_ex = max(_rn32_div(max(abs(x) for x in row), 448), fl)
        assert f32_bits(sk[0, n].item()) == f32_bits(s_ex)
        want = [e4m3_code(min(Fraction(_rn32_div(x, s_ex)), Fraction(448))) for x in row]
        assert k8[0, n].view(torch.uint8).tolist() == want
        vrow = [float(x) for x in vr[0, n].float().tolist()]
        sv_ex = max(_rn32_div(max(abs(x) for x in vrow), 448), fl)
        assert f32_bits(sv[0, n].item()) == f32_bits(sv_ex)
        wantv = [e4m3_code(min(Fraction(_rn32_div(x, sv_ex)), Fraction(448))) for x in vrow]
        assert v8t[0, :, n].contiguous().view(torch.uint8).tolist() == wantv
    assert (sv[0, 20:] == 0).all() and (v8t[0, :, 20:].view(torch.uint8) == 0).all()


@pytest.mark.parametrize("d", [128, 64])
def test_quant_q_exact_small(d):
    # Q uses a multiplication by the correctly rounded reciprocal (`sk1_t6i.hip:108`, `:115`).
    q, k, v = make_qkv(1, 1, 24, seed=9, std=1.3, d=d)
    qr = q.reshape(1, 24, d)
    sm = d ** -0.5
    for int8 in (True, False):
        q8, sq, cq = oracle.quant_q(qr, sm, int8=int8)
        top = 127 if int8 else 448
        smlog = rn32(Fraction(float(np.float32(sm))) * Fraction(float(np.float32(1.4426950408889634))))
        for n in range(24):
            row = [float(x) for x in qr[0, n].float().tolist()]
            amax = max(max(abs(x) for x in row), float(np.float32(1e-12)))
            qinv = _rn32_div(top, amax)
            s_ex = _rn32_div(amax, top)
            assert f32_bits(sq[0, n].item()) == f32_bits(s_ex)
            assert f32_bits(cq[0, n].item()) == f32_bits(rn32(Fraction(smlog) * Fraction(s_ex)))
            prod = [rn32(Fraction(x) * Fraction(qinv)) for x in row]
            if int8:
                assert q8[0, n].tolist() == [max(-128, min(127, rne_int(p))) for p in prod]
            else:
                want = [e4m3_code(max(min(Fraction(p), Fraction(448)), Fraction(-448))) for p in prod]
                assert q8[0, n].view(torch.uint8).tolist() == want


def test_kseq_mean_matches_fsum_and_is_order_free():
    q, k, v = make_qkv(1, 3, 301, seed=2, k_offset_std=2.0)
    kr = k.reshape(3, 301, 128)
    mean = oracle.kseq_mean(kr)
    for bh in range(3):
        for d in (0, 17, 127):
            col = [float(x) for x in kr[bh, :, d].float().tolist()]
            s = math.fsum(col)                        # exact here: the sum is representable
            assert Fraction(s) == sum(Fraction(x) for x in col)
            want = float(np.float32(s / 301.0))      # RN64 of s/N, then RN32 (the reference's)
            assert f32_bits(mean[bh, d].item()) == f32_bits(want)
    perm = torch.randperm(301, generator=torch.Generator().manual_seed(0))
    assert torch.equal(oracle.kseq_mean(kr[:, perm]), mean)


def test_fold_v_scale_closed_form():
    sv = torch.tensor([[0.5, 0.25, 0.0], [3.0, 1.5, 0.0]], dtype=torch.float32)
    s, svp = oracle.fold_v_scale(sv)
    assert s.tolist() == [1.0, 3.0]
    assert torch.equal(svp[0], sv[0])                  # S == 1: SV' is SV bit for bit
    assert f32_bits(svp[1, 1].item()) == f32_bits(rn32(Fraction(1.5) / 3))


# ----------------------------------------------------------------------------- attention
def _brute_force_row(q8r, cqr, k8, sk, v8t, svp, S, row, N, causal, int8, tile=64):
    """One output row of A.9-A.11 in numpy fp32 scalars with Python loops (no torch)."""
    f32 = np.float32
    n_pad = k8.shape[0]
    qv = q8r.astype(np.float64)
    m, l = f32(-np.inf), f32(0)
    acc = np.zeros(v8t.shape[0], dtype=np.float32)
    for j0 in range(0, n_pad, tile):
        s = []
        for n in range(j0, j0 + tile):
            dot = f32(float(np.dot(qv, k8[n].astype(np.float64))))
            val = f32(dot * f32(cqr * sk[n]))
            dead = (n > row) if causal else (n >= N)
            s.append(f32(-np.inf) if dead else val)
        m_new = f32(max(m, max(s)))
        m_use = f32(0) if m_new == -np.inf else m_new
        alpha = f32(2.0 ** float(f32(m - m_use)))
        p = [f32(2.0 ** float(f32(x - m_use))) for x in s]
        psum = f32(0)
        for x in p:
            psum = f32(psum + x)
        l = f32(f32(l * alpha) + psum)
        acc = (acc * alpha).astype(np.float32)
        for i, n in enumerate(range(j0, j0 + tile)):
            p8 = float(e4m3_value(e4m3_code(Fraction(float(f32(p[i] * f32(svp[n] * f32(448))))))))
            acc = (acc + np.float32(p8) * v8t[:, n].astype(np.float32)).astype(np.float32)
        m = m_new
    inv = f32(S / f32(l * f32(448))) if l > 0 else f32(0)
    return (acc * inv).astype(np.float32)


@pytest.mark.parametrize("d", [128, 64])
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("N", [5, 64, 130])
def test_attention_tiles_vs_brute_force(N, causal, d):
    q, k, v = make_qkv(1, 1, N, seed=N, k_offset_std=1.0, d=d)
    r = oracle.emulate_sageattn(q, k, v, is_causal=causal)
    k8 = r["k8"][0].numpy().astype(np.int32)
    v8t = r["v8t"][0].float().numpy()
    q8 = r["q8"][0].numpy().astype(np.int32)
    out = r["o"][0, 0].float().numpy()
    for row in sorted({0, 1, N // 2, N - 1}):
        want = _brute_force_row(q8[row], r["c_q"][0, row].item(), k8, r["sk"][0].numpy(), v8t,
                                r["svp"][0].numpy(), r["s"][0].item(), row, N, causal, True)
        got = out[row]
        assert np.allclose(got, want.astype(np.float16).astype(np.float32), rtol=2e-3, atol=2e-4), row


def test_causal_first_row_closed_form():
    # Row 0 of a causal call sees only key 0: p = exp2(0) = 1 exactly, so
    # O[0] = fp16( e4m3(RN(SV'[0]*448)) * V8[0] * RN(S / RN(1*448)) ).
    q, k, v = make_qkv(1, 2, 70, seed=4)
    v[0, 1, 0] *= 3000.0                       # plane 1: |V| > 448, so S > 1 there
    r = oracle.emulate_sageattn(q, k, v, is_causal=True)
    for bh in range(2):
        svp0, S = Fraction(r["svp"][bh, 0].item()), Fraction(r["s"][bh].item())
        p8 = e4m3_value(e4m3_code(rn32(rn32(svp0 * 448))))
        inv = rn32(S / rn32(Fraction(448)))
        v8 = [e4m3_value(c) for c in r["v8t"][bh, :, 0].contiguous().view(torch.uint8).tolist()]
        want = torch.tensor([rn32(rn32(p8 * x) * Fraction(inv)) for x in v8]).half()
        assert torch.equal(r["o"][0, bh, 0], want)
    assert r["s"][1].item() > 1.0


def test_uniform_keys_give_the_mean_of_v():
    # Identical keys: every score is equal, so the output is the (quantized) mean of V.
    q, k, v = make_qkv(1, 1, 200, seed=6)
    k[:] = k[:, :, :1]
    r = oracle.emulate_sageattn(q, k, v, is_causal=False, smooth_k=False)
    mean_v = v[0, 0].float().mean(0)
    assert (r["o"][0, 0].float() - mean_v).abs().max().item() < 0.02


# ----------------------------------------------------------------------------- logsumexp
def _scores_fp32(q8r, cqr, k8, sk, row, N, causal):
    """The emulated scores of one row (A.9) as fp32 scalars, masked keys dropped."""
    f32 = np.float32
    out = []
    for n in range(k8.shape[0]):
        dead = (n > row) if causal else (n >= N)
        if dead:
            continue
        dot = f32(float(np.dot(q8r.astype(np.float64), k8[n].astype(np.float64))))
        out.append(float(f32(dot * f32(cqr * sk[n]))))
    return out


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("N", [5, 64, 130])
def test_lse_vs_brute_force(N, causal):
    # log2 sum exp2 of the row's scores straight from their definition (fp64, no tiles, no
    # running max) against the tiled bookkeeping m_use + log2(l).
    q, k, v = make_qkv(1, 1, N, seed=N + 1, k_offset_std=1.0)
    r = oracle.emulate_sageattn(q, k, v, is_causal=causal, smooth_k=False)
    k8 = r["k8"][0].numpy().astype(np.int32)
    q8 = r["q8"][0].numpy().astype(np.int32)
    for row in sorted({0, 1, N // 2, N - 1}):
        sc = _scores_fp32(q8[row], r["c_q"][0, row].item(), k8, r["sk"][0].numpy(), row, N, causal)
        mx = max(sc)
        lse2 = mx + math.log2(sum(2.0 ** (x - mx) for x in sc))
        got = r["lse"][0, 0, row].item()
        assert abs(got - lse2 / 1.44269504) < 2e-5 * max(1.0, abs(got)), (row, got, lse2)


def test_lse_causal_first_row_closed_form():
    # Row 0 of a causal call sees only key 0: m = s[0,0], l = 1, so lse = s[0,0] / 1.44269504
    # (+ the smooth_k correction sm_scale * q[0] . mean).
    q, k, v = make_qkv(1, 2, 70, seed=9, k_offset_std=2.0)
    r = oracle.emulate_sageattn(q, k, v, is_causal=True, smooth_k=True)
    for bh in range(2):
        s00 = _scores_fp32(r["q8"][bh, 0].numpy().astype(np.int32), r["c_q"][bh, 0].item(),
                           r["k8"][bh].numpy().astype(np.int32), r["sk"][bh].numpy(), 0, 70, True)
        assert len(s00) == 1
        corr = float(torch.dot(q[0, bh, 0].float(), r["mean"][bh]).item()) * r["sm_scale"]
        want = s00[0] / 1.44269504 + corr
        assert abs(r["lse"][0, bh, 0].item() - want) < 1e-4, (bh, r["lse"][0, bh, 0].item(), want)


def test_lse_uniform_keys_closed_form():
    # Identical keys: every score of a row equals c, so lse = (c + log2(N)) / 1.44269504.
    N = 200
    q, k, v = make_qkv(1, 1, N, seed=6)
    k[:] = k[:, :, :1]
    r = oracle.emulate_sageattn(q, k, v, is_causal=False, smooth_k=False)
    for row in (0, 17, N - 1):
        c = _scores_fp32(r["q8"][0, row].numpy().astype(np.int32), r["c_q"][0, row].item(),
                         r["k8"][0].numpy().astype(np.int32), r["sk"][0].numpy(), row, N, False)
        assert len(set(c)) == 1
        want = (c[0] + math.log2(N)) / 1.44269504
        assert abs(r["lse"][0, 0, row].item() - want) < 1e-4


def test_lse_close_to_exact_and_needs_the_correction():
    # With a K channel offset (mean ~ N(0, 2)), smoothing shifts every score of a row by
    # sm_scale * q . mean; the corrected logsumexp must track the unquantized one, and the same
    # value without the correction must not.
    q, k, v = make_qkv(1, 2, 300, seed=12, k_offset_std=2.0)
    for causal in (False, True):
        r = oracle.emulate_sageattn(q, k, v, is_causal=causal, smooth_k=True)
        ex = oracle.exact_lse(q, k, is_causal=causal).float()
        err = (r["lse"] - ex).abs()
        assert err.max().item() < 0.05, err.max().item()
        corr = torch.matmul(q[0].float(), r["mean"][:, :, None]).squeeze(-1) * r["sm_scale"]
        assert (r["lse"][0] - corr - ex[0]).abs().max().item() > 0.5


@pytest.mark.parametrize("d", [128, 64])
def test_emulation_close_to_exact_attention(d):
    # The scheme's error against exact attention on N(0,1) inputs: the reference's bar is 0.08
    # relative RMS (`tests/test_sk1_backend.py:28-29`), observed 0.03-0.055.
    for dtype in (torch.float16, torch.bfloat16):
        q, k, v = make_qkv(1, 4, 512, seed=1, dtype=dtype, d=d)
        for causal in (False, True):
            o = oracle.emulate_sageattn(q, k, v, is_causal=causal)["o"].double()
            ex = oracle.exact_attention(q, k, v, is_causal=causal)
            rel = ((o - ex).pow(2).mean().sqrt() / ex.pow(2).mean().sqrt()).item()
            assert rel < 0.08, (dtype, causal, rel)


MUTATIONS = {
    # name: (exact source text in attention_tiles, its planted replacement, causal)
    "causal_mask_off_by_one": ("(keys > rows) if causal", "(keys >= rows) if causal", True),
    "tail_mask_off_by_one": ("else (keys >= N)", "else (keys > N)", False),
    "l_not_rescaled": ("l = l * alpha + p.sum(dim=2)", "l = l + p.sum(dim=2)", True),
    "acc_not_rescaled": ("acc = acc * alpha[:, :, None] +", "acc = acc +", False),
    "fold_dropped": ("p8 = (p * sv448[:, None, ks])", "p8 = (p * P_SCALE)", True),
    "keys_reversed_in_tile": ("torch.matmul(qf, kf[:, ks].transpose(1, 2))",
                              "torch.matmul(qf, kf[:, ks].flip(1).transpose(1, 2))", False),
}


def _mutated_attention_tiles(old, new):
    import inspect
    import oracle.sage_scheme as mod
    src = inspect.getsource(mod.attention_tiles)
    assert src.count(old) == 1, old
    ns = dict(vars(mod))
    exec(compile(src.replace(old, new), "<planted>", "exec"), ns)
    return ns["attention_tiles"]


@pytest.mark.parametrize("name", sorted(MUTATIONS))
def test_planted_mistakes_are_caught(name, monkeypatch):
    # Each plausible slip, planted into a copy of the oracle's attention loop, must make the
    # brute-force pin fail on at least one row (and the unmutated oracle passes the same check).
    import oracle.sage_scheme as mod
    old, new, causal = MUTATIONS[name]
    N = 130
    q, k, v = make_qkv(1, 1, N, seed=21, k_offset_std=1.0)
    v[0, 0, 3, :5] = 900.0                       # S > 1, so a dropped fold changes the output

    def mismatched_rows(fn):
        monkeypatch.setattr(mod, "attention_tiles", fn)
        r = mod.emulate_sageattn(q, k, v, is_causal=causal)
        k8 = r["k8"][0].numpy().astype(np.int32)
        v8t = r["v8t"][0].float().numpy()
        q8 = r["q8"][0].numpy().astype(np.int32)
        out = r["o"][0, 0].float().numpy()
        bad = 0
        for row in (0, 1, 64, N - 1):
            want = _brute_force_row(q8[row], r["c_q"][0, row].item(), k8, r["sk"][0].numpy(), v8t,
                                    r["svp"][0].numpy(), r["s"][0].item(), row, N, causal, True)
            want = want.astype(np.float16).astype(np.float32)
            if not np.allclose(out[row], want, rtol=2e-3, atol=2e-4, equal_nan=False):
                bad += 1
        return bad

    original = mod.attention_tiles
    assert mismatched_rows(original) == 0
    assert mismatched_rows(_mutated_attention_tiles(old, new)) > 0, name


def test_fp16_rounded_probabilities_fail_the_regression_bar(monkeypatch):
    # The GPU tests hold outputs to the north star's rel-L1 <= 1e-2 tightened to the regression
    # bar of their Q.K form (sage_testutil.REL_L1_REGRESSION). A per-score chain that rounds p at
    # fp16 level, planted here into a copy of the oracle's loop, stays inside 1e-2 but not inside
    # the int8 bar: about 1 % of its e4m3 P codes cross a rounding boundary.
    import oracle.sage_scheme as mod
    from sage_testutil import REL_L1_MAX, rel_l1, rel_l1_bar
    q, k, v = make_qkv(1, 2, 1024, seed=3, k_offset_std=2.0)
    ref = mod.emulate_sageattn(q, k, v)["o"]
    monkeypatch.setattr(mod, "attention_tiles", _mutated_attention_tiles(
        "p = torch.exp2(s - m_use[:, :, None])",
        "p = torch.exp2(s - m_use[:, :, None]).half().float()"))
    rl = rel_l1(mod.emulate_sageattn(q, k, v)["o"], ref)
    assert rel_l1_bar(True) < rl < REL_L1_MAX, rl


def test_nhd_layout_is_a_view():
    q, k, v = make_qkv(2, 3, 100, seed=1)
    a = oracle.emulate_sageattn(q, k, v, is_causal=True)["o"]
    qn, kn, vn = (t.transpose(1, 2).contiguous() for t in (q, k, v))
    b = oracle.emulate_sageattn(qn, kn, vn, tensor_layout="NHD", is_causal=True)["o"]
    assert torch.equal(b.transpose(1, 2), a)


# ----------------------------------------------------------------------------- GQA, kv length
def test_exact_attention_gqa_and_kv_length_match_torch_sdpa():
    # The yardstick's head map and key length against torch's own SDPA (enable_gqa repeats each
    # K/V head over its group of H // H_kv query heads), fp64 on the CPU.
    sdpa = torch.nn.functional.scaled_dot_product_attention
    for (h, hk, n, nk, causal) in ((6, 2, 40, 40, True), (6, 3, 17, 90, False), (4, 1, 70, 9, False)):
        q, k, v = make_qkv(2, h, n, seed=h + nk, h_kv=hk, n_kv=nk)
        want = sdpa(q.double(), k.double(), v.double(), is_causal=causal, enable_gqa=True)
        got = oracle.exact_attention(q, k, v, is_causal=causal)
        assert torch.allclose(got, want, rtol=1e-10, atol=1e-12)
        s = torch.matmul(q.double(), k.double().repeat_interleave(h // hk, 1).transpose(2, 3))
        s = s * q.shape[-1] ** -0.5
        if causal:
            s = s.masked_fill(torch.ones(n, nk, dtype=torch.bool).triu(1), -math.inf)
        assert torch.allclose(oracle.exact_lse(q, k, is_causal=causal), torch.logsumexp(s, -1))


def test_gqa_equals_repeated_kv_heads():
    # Grouped K/V heads are, by definition, each K/V head repeated over its group: the emulation
    # with H_kv heads must give the bits of the emulation on explicitly repeated K/V (per-token
    # quantization, the per-plane mean and the per-plane fold are all unchanged by the repeat).
    for dtype in (torch.float16, torch.bfloat16):
        q, k, v = make_qkv(2, 6, 100, seed=8, dtype=dtype, h_kv=2, k_offset_std=1.5)
        a = oracle.emulate_sageattn(q, k, v, is_causal=True)
        b = oracle.emulate_sageattn(q, k.repeat_interleave(3, 1), v.repeat_interleave(3, 1),
                                    is_causal=True)
        assert torch.equal(a["o"], b["o"]) and torch.equal(a["lse"], b["lse"])
        assert a["k8"].shape[0] == 4 and b["k8"].shape[0] == 12
        # the map matters: heads of different groups see different K/V
        assert not torch.equal(a["o"][:, 0], a["o"][:, 3])


def test_kv_plane_map_and_refusals():
    assert oracle.kv_planes(2, 6, 2, 5, 5, True).tolist() == [0, 0, 0, 1, 1, 1, 2, 2, 2, 3, 3, 3]
    assert oracle.kv_planes(1, 4, 4, 5, 9, False).tolist() == [0, 1, 2, 3]
    assert oracle.kv_planes(1, 4, 1, 5, 9, False).tolist() == [0, 0, 0, 0]
    with pytest.raises(ValueError):
        oracle.kv_planes(1, 6, 4, 5, 5, False)
    with pytest.raises(ValueError):
        oracle.kv_planes(1, 4, 4, 5, 9, True)


@pytest.mark.parametrize("nq,nk", [(5, 130), (130, 5), (64, 200)])
def test_kv_length_rows_are_independent_of_q_length(nq, nk):
    # With its own key length, each query row sees all N_kv keys: the emulation of a few rows
    # equals those rows of a longer call on the same K/V (a key mask taken from the query length
    # would drop or invent keys), and every row matches the brute-force restatement.
    q, k, v = make_qkv(1, 1, max(nq, 140), seed=nq + nk, n_kv=nk, k_offset_std=1.0)
    full = oracle.emulate_sageattn(q, k, v)
    part = oracle.emulate_sageattn(q[:, :, :nq], k, v)
    assert torch.equal(part["o"], full["o"][:, :, :nq])
    assert torch.equal(part["lse"], full["lse"][:, :, :nq])
    r = part
    k8 = r["k8"][0].numpy().astype(np.int32)
    v8t = r["v8t"][0].float().numpy()
    q8 = r["q8"][0].numpy().astype(np.int32)
    out = r["o"][0, 0].float().numpy()
    for row in sorted({0, nq // 2, nq - 1}):
        want = _brute_force_row(q8[row], r["c_q"][0, row].item(), k8, r["sk"][0].numpy(), v8t,
                                r["svp"][0].numpy(), r["s"][0].item(), row, nk, False, True)
        assert np.allclose(out[row], want.astype(np.float16).astype(np.float32), rtol=2e-3,
                           atol=2e-4), row


def test_gqa_and_kv_length_close_to_exact_attention():
    for dtype in (torch.float16, torch.bfloat16):
        q, k, v = make_qkv(1, 8, 300, seed=2, dtype=dtype, h_kv=2, n_kv=515)
        o = oracle.emulate_sageattn(q, k, v)["o"].double()
        ex = oracle.exact_attention(q, k, v)
        rel = ((o - ex).pow(2).mean().sqrt() / ex.pow(2).mean().sqrt()).item()
        assert rel < 0.08, (dtype, rel)


# ----------------------------------------------------------------------------- smooth_v
def test_reference_fp32_chunked_mean_exact_on_integer_data():
    # integer-valued rows: every fp32 partial sum is exact, so the reference's fp32 chunked mean
    # (quant_triton.py:303-373) is RN32(sum / N), the correctly rounded mean -- the same bits as
    # the fp64 mean this build uses, at lengths across chunk and 16-row group boundaries
    g = torch.Generator().manual_seed(5)
    for n in (1, 15, 16, 17, 1023, 1024, 1025, 3000):
        x = torch.randint(-64, 65, (2, n, 8), generator=g).to(torch.float16)
        a = oracle.vseq_mean_fp32_chunked(x)
        b = oracle.kseq_mean(x)
        want = torch.tensor([[float(np.float32(math.fsum(x[i, :, d].double().tolist()) / n))
                              for d in range(8)] for i in range(2)], dtype=torch.float32)
        assert torch.equal(a, want) and torch.equal(b, want), n


def test_reference_fp32_chunked_mean_order_by_brute_force():
    # a chunk is a sequence of 16-row group sums (each a pairwise tree), added in row order; the
    # chunk partials are then added in chunk order and divided once, all in fp32 -- restated
    # scalar by scalar with numpy fp32 on a small case (chunk 32, so three partial chunks)
    g = torch.Generator().manual_seed(6)
    x = (torch.randn(1, 70, 3, generator=g) * 1e3).to(torch.float16)
    got = oracle.vseq_mean_fp32_chunked(x, chunk=32)
    xf = x.float().numpy()
    for d in range(3):
        parts = []
        for c in range(3):
            acc = np.float32(0)
            for r in range(32 * c, 32 * c + 32, 16):
                vals = [xf[0, i, d] if i < 70 else np.float32(0) for i in range(r, r + 16)]
                while len(vals) > 1:
                    vals = [np.float32(vals[i] + vals[i + 1]) for i in range(0, len(vals), 2)]
                acc = np.float32(acc + vals[0])
            parts.append(acc)
        tot = np.float32(0)
        for p_ in parts:
            tot = np.float32(tot + p_)
        assert f32_bits(got[0, d].item()) == f32_bits(float(np.float32(tot / np.float32(70))))


def _fp32_chunked_mean_exact(x, chunk=1024, group=16, chunk_order=1, divide="div"):
    """The reference's fp32 chunked mean (`quant_triton.py:303-343`) in exact rational arithmetic,
    each fp32 operation one `rn32`: per chunk of `chunk` rows an accumulator starting at 0 receives
    the `group`-row sums in row order, the chunk partials are added in chunk order (reversed with
    `chunk_order=-1`), then one division by N. Group sums are formed exactly and rounded once,
    which is every order's result when, as on `_exact_group_data`, each one is representable.
    `divide`: "div" (the reference), "recip" (times RN(1/N)), "pad" (by the padded length), "f64"
    (the fp32 sum divided in fp64, then rounded to fp32)."""
    N, D = x.shape
    out = []
    for c in range(D):
        col = [Fraction(float(v)) for v in x[:, c]]
        parts = []
        for c0 in range(0, N, chunk):
            acc = Fraction(0)
            for g0 in range(c0, c0 + chunk, group):
                gs = sum(col[g0:min(g0 + group, N)], Fraction(0)) if g0 < N else Fraction(0)
                acc = Fraction(rn32(acc + Fraction(rn32(gs))))
            parts.append(acc)
        tot = Fraction(0)
        for p_ in parts[::chunk_order]:
            tot = Fraction(rn32(tot + p_))
        if divide == "f64":
            out.append(float(np.float32(np.float64(float(tot)) / np.float64(N))))
            continue
        den = {"div": Fraction(N), "pad": Fraction(len(parts) * chunk)}.get(divide)
        out.append(rn32(tot / den) if den is not None
                   else rn32(tot * Fraction(rn32(Fraction(1, N)))))
    return out


def _exact_group_data(seed, N, D):
    """fp16 columns whose every 16-row group is all zeros, all one value with at most 3 significant
    bits (1024 .. 3584, either sign), or a single nonzero row 1 + k/1024 (k odd): every partial sum
    inside a group, in any order, is exact in fp32, so Triton's unspecified order inside one
    `tl.sum` cannot change a bit, while the fp32 `acc +=` across groups (magnitudes up to ~2^21
    against fine bits at 2^-10) and across chunks must round."""
    rng = np.random.default_rng(seed)
    x = np.zeros((N, D), dtype=np.float16)
    for c in range(D):
        for g0 in range(0, N, 16):
            kind = rng.integers(0, 3)
            if kind == 1:
                x[g0:g0 + 16, c] = float(rng.choice([1024., 1536., 2048., 3072., 3584.])) \
                    * float(rng.choice([-1, 1]))
            elif kind == 2:
                r = g0 + int(rng.integers(0, 16))
                if r < N:
                    x[r, c] = (1 + (2 * int(rng.integers(0, 512)) + 1) / 1024.0) \
                        * float(rng.choice([-1, 1]))
    for c in range(D):
        for g0 in range(0, N, 16):
            vals = {float(v) for v in x[g0:g0 + 16, c] if v != 0}
            assert len(vals) <= 1
            for v in vals:
                assert all(rn32(k * Fraction(v)) == k * Fraction(v) for k in range(17))
    return x


def test_reference_fp32_chunked_mean_pinned_where_fp32_rounding_decides():
    # The part of the reference's mean the reference fixes -- fp32 accumulation of 16-row group
    # sums in row order within 1024-row chunks, chunk partials in chunk order, one fp32 division
    # (quant_triton.py:303-343) -- on data where that accumulation must round and the order
    # inside a group cannot matter (three chunks, a ragged last chunk and group). The oracle must
    # equal the exact simulation bit for bit, and each plausible slip must be caught.
    N, D = 2599, 16
    x = _exact_group_data(7, N, D)
    want = _fp32_chunked_mean_exact(x)
    got = oracle.vseq_mean_fp32_chunked(torch.from_numpy(x)[None])[0].tolist()
    assert [f32_bits(a) for a in got] == [f32_bits(a) for a in want]

    def caught(other):
        return sum(f32_bits(a) != f32_bits(b) for a, b in zip(want, other))
    xt = torch.from_numpy(x)
    # fp64 accumulation (the whole sum in fp64, or in fp64 per chunk), one rounding at the end
    assert caught((xt.double().sum(0) / N).float().tolist()) > 0
    per_chunk64 = sum(xt[c0:c0 + 1024].double().sum(0) for c0 in range(0, N, 1024))
    assert caught((per_chunk64 / N).float().tolist()) > 0
    assert caught([rn32(Fraction(math.fsum(float(v) for v in x[:, c])) / N)
                   for c in range(D)]) > 0
    assert caught(_fp32_chunked_mean_exact(x, chunk_order=-1)) > 0     # partials in another order
    assert caught(_fp32_chunked_mean_exact(x, chunk=512)) > 0          # another chunk length
    assert caught(_fp32_chunked_mean_exact(x, group=32)) > 0           # another group length
    assert caught(_fp32_chunked_mean_exact(x, divide="recip")) > 0     # times RN(1/N)
    assert caught(_fp32_chunked_mean_exact(x, divide="pad")) > 0       # by the padded length
    # The division done in fp64 and rounded to fp32 is not a slip: for fp32 operands it gives the
    # same bits as the fp32 division (double rounding is innocuous for +, -, *, / when the wider
    # format has at least 2p + 2 significand bits, 53 >= 2*24 + 2; Figueroa 1995), as here.
    assert caught(_fp32_chunked_mean_exact(x, divide="f64")) == 0


def test_fp64_mean_is_within_a_few_ulps_of_the_reference_fp32_mean():
    # the build's V mean (fp64 sums, one rounding) against the reference's fp32 chunked mean on
    # offset fp16 data at a long length: their difference is the fp32 summation error alone,
    # bounded by N * 2^-24 * (sum |v|) / N per channel, and the fp64 mean is the closer of the two
    # to the exact mean
    g = torch.Generator().manual_seed(7)
    n = 9000
    x = (torch.randn(2, n, 16, generator=g) + 3.0).to(torch.float16)
    a = oracle.vseq_mean_fp32_chunked(x).double()
    b = oracle.kseq_mean(x).double()
    exact = x.double().mean(dim=1)
    bound = n * 2.0 ** -24 * x.double().abs().mean(dim=1)
    assert ((a - b).abs() <= bound).all()
    assert ((b - exact).abs() <= (a - exact).abs() + 1e-12).all()


def test_smooth_v_mean_is_fsum_of_v_and_centering_precedes_the_scale():
    # V's mean is the same fp64 sequence mean as K's, and V is centred (fp32) before its absmax:
    # SV = max(RN(max_d |RN(v - mu)| / 448), 1e-12) on live rows, V8T the e4m3 of RN(RN(v - mu)/SV).
    q, k, v = make_qkv(1, 2, 77, seed=41)
    v = (v.float() + 3.0).half()                             # a per-channel offset
    r = oracle.emulate_sageattn(q, k, v, smooth_v=True, smooth_k=False)
    vr = v.reshape(2, 77, 128)
    for bh in range(2):
        for d in (0, 63, 127):
            col = [float(x) for x in vr[bh, :, d].float().tolist()]
            assert f32_bits(r["vmean"][bh, d].item()) == f32_bits(float(np.float32(math.fsum(col) / 77)))
        for n in (0, 40, 76):
            c = [np.float32(np.float32(x) - np.float32(r["vmean"][bh, d].item()))
                 for d, x in enumerate(vr[bh, n].float().tolist())]
            sv = max(np.float32(max(abs(x) for x in c) / np.float32(448)), np.float32(1e-12))
            assert f32_bits(r["sv"][bh, n].item()) == f32_bits(float(sv))
            want = [e4m3_code(min(Fraction(float(np.float32(x / sv))), Fraction(448))) for x in c]
            assert r["v8t"][bh, :, n].contiguous().view(torch.uint8).tolist() == want
        assert r["v8t"][bh, :, 77:].float().abs().max().item() == 0.0     # pad rows stay zero


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_smooth_v_identical_rows_give_the_row_exactly(dtype):
    # Every token's V equal to one vector c: the centred V is exactly 0, so the output is
    # T(RN(0 + mean)) = c bit for bit, for every query, whatever the scores are.
    q, k, v = make_qkv(2, 2, 90, seed=9, dtype=dtype)
    v[:] = v[:, :, :1]
    for causal in (False, True):
        o = oracle.emulate_sageattn(q, k, v, is_causal=causal, smooth_v=True)["o"]
        assert torch.equal(o, v.expand_as(o))
        o_plain = oracle.emulate_sageattn(q, k, v, is_causal=causal)["o"]
        assert not torch.equal(o_plain, v.expand_as(o))        # quantized V does not round-trip


@pytest.mark.parametrize("causal", [False, True])
def test_smooth_v_vs_brute_force(causal):
    N = 130
    q, k, v = make_qkv(1, 1, N, seed=17, k_offset_std=1.0)
    v = (v.float() * 0.5 + 2.5).half()
    r = oracle.emulate_sageattn(q, k, v, is_causal=causal, smooth_v=True)
    k8 = r["k8"][0].numpy().astype(np.int32)
    v8t = r["v8t"][0].float().numpy()
    q8 = r["q8"][0].numpy().astype(np.int32)
    out = r["o"][0, 0].float().numpy()
    vm = r["vmean"][0].numpy()
    for row in (0, 1, 64, N - 1):
        base = _brute_force_row(q8[row], r["c_q"][0, row].item(), k8, r["sk"][0].numpy(), v8t,
                                r["svp"][0].numpy(), r["s"][0].item(), row, N, causal, True)
        # the epilogue's fma(acc, inv, vm), from the brute-force acc*inv (one rounding apart)
        want = (base.astype(np.float64) + vm.astype(np.float64)).astype(np.float32)
        assert np.allclose(out[row], want.astype(np.float16).astype(np.float32), rtol=2e-3,
                           atol=2e-3), row


def test_smooth_v_wins_on_offset_v_and_the_add_back_is_needed(monkeypatch):
    # The reference's finding (docs/FINDINGS.md F005): with a per-channel V offset of 6, centring
    # before the per-token scale is far more accurate. A dropped add-back fails the same check.
    import oracle.sage_scheme as mod
    q, k, v = make_qkv(1, 2, 400, seed=5)
    off = torch.randn(1, 2, 1, 128, generator=torch.Generator().manual_seed(3)) * 6.0
    v = (v.float() * 0.3 + off).half()
    ex = oracle.exact_attention(q, k, v)
    err_plain = (oracle.emulate_sageattn(q, k, v)["o"].double() - ex).abs().max().item()
    err_sv = (oracle.emulate_sageattn(q, k, v, smooth_v=True)["o"].double() - ex).abs().max().item()
    assert err_sv * 10 < err_plain, (err_sv, err_plain)

    import inspect
    src = inspect.getsource(mod.attention_tiles)
    old = "+ vmean.double()[:, None, :]"
    assert src.count(old) == 1
    ns = dict(vars(mod))
    exec(compile(src.replace(old, ""), "<planted>", "exec"), ns)
    monkeypatch.setattr(mod, "attention_tiles", ns["attention_tiles"])
    err_planted = (mod.emulate_sageattn(q, k, v, smooth_v=True)["o"].double() - ex).abs().max().item()
    assert err_planted > 1.0


# ----------------------------------------------------------------------------- row subsets
@pytest.mark.parametrize("causal", [True, False])
def test_row_subset_equals_the_full_emulation(causal):
    """`attention_tiles(..., row0=r)` over a slice of query rows gives those rows of the whole
    emulation bit for bit (the long-sequence GPU test checks only a few rows this way)."""
    N = 300
    q, k, v = make_qkv(1, 1, N, seed=11, k_offset_std=2.0)
    full = oracle.emulate_sageattn(q, k, v, is_causal=causal)["o"][0, 0]
    kr, vr = k[0], v[0]
    n_pad = oracle.n_pad_for(N)
    k8, sk = oracle.quant_k(kr, n_pad, mean=oracle.kseq_mean(kr), int8=True)
    v8t, sv = oracle.quant_v(vr, n_pad)
    s, svp = oracle.fold_v_scale(sv)
    for r0, r1 in ((0, 7), (100, 165), (N - 64, N)):
        q8, _, cq = oracle.quant_q(q[0][:, r0:r1], 128 ** -0.5, int8=True)
        part = oracle.attention_tiles(q8, cq, k8, sk, v8t, svp, s, N, causal, q.dtype, row0=r0)
        assert torch.equal(part[0], full[r0:r1]), (r0, r1)


@pytest.mark.parametrize("causal,smooth_v,layout", [(True, False, "HND"), (False, True, "NHD")])
def test_emulate_rows_equals_the_full_emulation(causal, smooth_v, layout):
    """The row-slice emulation used by the large GPU sweep gives the full emulation's rows and
    logsumexp bit for bit, with grouped K/V heads, a key length of their own and smooth_v."""
    from sage_testutil import emulate_rows
    N = 200
    q, k, v = make_qkv(2, 4, N, seed=5, k_offset_std=2.0, layout=layout, h_kv=2,
                       n_kv=N if causal else 150, v_offset_std=1.0)
    full = oracle.emulate_sageattn(q, k, v, tensor_layout=layout, is_causal=causal,
                                   smooth_v=smooth_v)
    o_full = oracle.to_hnd(full["o"], layout)
    for r in (range(0, 64), range(70, 133), range(N - 64, N)):
        o, lse = emulate_rows(q, k, v, r, tensor_layout=layout, is_causal=causal,
                              smooth_v=smooth_v)
        assert torch.equal(o, o_full[:, :, r.start:r.stop]), r
        assert torch.equal(lse, full["lse"][:, :, r.start:r.stop]), r
