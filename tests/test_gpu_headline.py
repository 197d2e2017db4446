"""Parity at the benchmark's own sequence lengths (GPU tests), one head each so that the CPU
emulation finishes in seconds: the headline c3c (fp16, N = 47520, causal, int8 Q.K, the 256-query
kernel) and c4 (bf16, N = 16384, causal, e4m3 Q.K, the 128-query kernel), on the configurations'
synthetic inputs. The prologue's quantized tensors must equal the oracle's byte for byte and the
output must reach cos >= 0.999 and rel-L1 <= 1e-2 against the emulation.
"""
import pytest
import torch

import oracle
from parity_report import quantized_bit_exact
from sage_testutil import cosine, have_gfx950, make_qkv, rel_l1

pytestmark = [pytest.mark.gpu,
              pytest.mark.skipif(not have_gfx950(), reason="needs a gfx950 GPU")]


@pytest.mark.parametrize("name,dtype,N,outliers,std", [
    ("c3c", torch.float16, 47520, 0.0, 1.0),
    ("c4", torch.bfloat16, 16384, 0.001, 1.5),
])
def test_benchmark_length_parity(name, dtype, N, outliers, std):
    from sageattention import sageattn
    q, k, v = make_qkv(1, 1, N, seed=0, dtype=dtype, std=std, k_offset_std=2.0,
                       outlier_frac=outliers)
    print("case", name, N, flush=True)
    assert quantized_bit_exact(k, v, "HND", k_int8=(dtype == torch.float16))
    out = sageattn(q.cuda(), k.cuda(), v.cuda(), tensor_layout="HND", is_causal=True)
    torch.cuda.synchronize()
    emu = oracle.emulate_sageattn(q, k, v, is_causal=True)["o"]
    out = out.cpu()
    assert torch.isfinite(out).all()
    c, r = cosine(out, emu), rel_l1(out, emu)
    assert c >= 0.999 and r <= 1e-2, (c, r)
