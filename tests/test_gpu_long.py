"""A sequence far beyond the benchmark's (GPU): N = 262161 (5.5x the headline), one head.

At this length the staging offsets inside a plane reach 128 x N_pad = 33.6 M bytes, and the causal
grid has 2049 query tiles per plane. Checked with properties that do not need the whole emulation:
* the prologue's quantized tensors equal the oracle's byte for byte (the oracle's quantizers are
  vectorized and run at this size in seconds);
* the last 128 query rows (the longest causal rows: every key) and the first 64 equal the
  emulation's at the usual bars, computed for those rows alone (rows are independent);
* the 128-query, pipelined and 256-query kernels agree bit for bit, and NHD equals HND;
* at head_dim 64 (non-causal), the key split over 4097 key blocks (2049 and 2048 per wave pair)
  meets the same bars on the same rows and stays within rounding of the pipelined kernel.
"""
import pytest
import torch

import oracle
from sage_testutil import (cosine, have_gfx950, make_qkv, quantized_bit_exact, rel_l1,
                           rel_l1_bar)

pytestmark = [pytest.mark.gpu,
              pytest.mark.skipif(not have_gfx950(), reason="needs a gfx950 GPU")]

N_LONG = 262161


def _rows_emulated(q, k, v, rows, causal):
    """The emulation's output for the query rows `rows` (a range) of plane 0."""
    kr, vr = k[0], v[0]
    N, D = kr.shape[1], kr.shape[2]
    n_pad = oracle.n_pad_for(N)
    mean = oracle.kseq_mean(kr)
    k8, sk = oracle.quant_k(kr, n_pad, mean=mean, int8=True)
    v8t, sv = oracle.quant_v(vr, n_pad)
    s, svp = oracle.fold_v_scale(sv)
    q8, sq, cq = oracle.quant_q(q[0][:, rows.start:rows.stop], D ** -0.5, int8=True)
    return oracle.attention_tiles(q8, cq, k8, sk, v8t, svp, s, N, causal, q.dtype,
                                  row0=rows.start)


@pytest.mark.parametrize("causal", [True, False])
def test_long_sequence(causal):
    from sageattention import sageattn
    from sageattention.sk1_backend import sk1_forward
    from sageattention.sk1_backend.sk1_loader import SageLib
    N = N_LONG
    print("long N", N, "causal", causal, flush=True)
    q, k, v = make_qkv(1, 1, N, seed=7, dtype=torch.float16, k_offset_std=2.0, outlier_frac=1e-4)
    if causal:
        assert quantized_bit_exact(k, v, "HND", k_int8=True)
    out = sageattn(q.cuda(), k.cuda(), v.cuda(), is_causal=causal)
    torch.cuda.synchronize()
    out = out.cpu()
    assert torch.isfinite(out).all()
    for rows in (range(N - 128, N), range(0, 64)):
        ref = _rows_emulated(q, k, v, rows, causal)
        got = out[0, 0, rows.start:rows.stop]
        c, r = cosine(got, ref[0]), rel_l1(got, ref[0])
        assert c >= 0.999 and r <= rel_l1_bar(True), (rows, c, r)
    lib = SageLib.get()
    for kern in (1, 2, 3):
        o = sk1_forward(lib, q.cuda(), k.cuda(), v.cuda(), is_causal=causal, kernel=kern)
        torch.cuda.synchronize()
        assert torch.equal(o.cpu(), out), kern
    if causal:
        o_nhd = sageattn(q.transpose(1, 2).contiguous().cuda(), k.transpose(1, 2).contiguous().cuda(),
                         v.transpose(1, 2).contiguous().cuda(), tensor_layout="NHD", is_causal=True)
        torch.cuda.synchronize()
        assert torch.equal(o_nhd.cpu().transpose(1, 2), out)


def test_long_sequence_head_dim_64_key_split():
    from sageattention.sk1_backend import sk1_forward
    from sageattention.sk1_backend.sk1_loader import SageLib
    N = N_LONG
    print("long N", N, "head_dim 64 key split", flush=True)
    q, k, v = make_qkv(1, 1, N, seed=9, dtype=torch.float16, k_offset_std=2.0, outlier_frac=1e-4,
                       d=64)
    lib = SageLib.get()
    outs = {}
    for kern in (3, 4):
        outs[kern] = sk1_forward(lib, q.cuda(), k.cuda(), v.cuda(), kernel=kern).cpu()
        torch.cuda.synchronize()
        assert torch.isfinite(outs[kern]).all()
    for rows in (range(N - 128, N), range(0, 64)):
        ref = _rows_emulated(q, k, v, rows, False)
        for kern in (3, 4):
            got = outs[kern][0, 0, rows.start:rows.stop]
            c, r = cosine(got, ref[0]), rel_l1(got, ref[0])
            assert c >= 0.999 and r <= rel_l1_bar(True), (kern, rows, c, r)
    err = (outs[4].float() - outs[3].float()).abs()
    assert (err <= 2 * 2.0 ** -10 * outs[3].float().abs() + 1e-5 * v.float().abs().max()).all()
