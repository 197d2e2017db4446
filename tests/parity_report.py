"""Accuracy report of the GPU path at every benchmark configuration's sequence length (GPU box).

    python tests/parity_report.py [--heads-cap 4]

For each configuration of the benchmark (fp16 and bf16, causal and not, the short and batched
calls) the inputs are the configuration's synthetic ones at its real N, with the head count capped
so that the CPU references finish in minutes. One line per case:

* whether the prologue's quantized tensors and scales (mu, K8, SK, V8T, SV', S) equal the oracle's
  byte for byte;
* `cos`, `rel_l1`: the output of `sageattn` (through the C ABI on cuda:0) against the CPU emulation
  of the reference scheme (`oracle.emulate_sageattn`), the bar being cos >= 0.999 and
  rel-L1 <= 1e-2;
* `emu_rel_rms`, `gpu_rel_rms`: the emulation's and the GPU output's relative RMS error against
  exact attention (`oracle.exact_attention`, fp64 on the CPU, chunked), i.e. the scheme's own
  quantization error and the GPU path's, which the reference's tests bound by 0.08
  (tests/test_sk1_backend.py:29 of the reference).

Test infrastructure: it imports the oracle as the checker; the product path it measures is the
HIP library.
"""
import argparse
import os
import sys
import time

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
for p in (ROOT, os.path.join(ROOT, "sageattention-rdna4_amd"), HERE):
    if p not in sys.path:
        sys.path.insert(0, p)

import torch  # noqa: E402

import oracle  # noqa: E402
from sage_testutil import bytes_equal, cosine, make_qkv, rel_l1, rel_rms  # noqa: E402


def quantized_bit_exact(k, v, layout, k_int8):
    """The prologue's mu, K8, SK, V8T, SV' and S through the C ABI against the oracle's: True when
    every byte matches (outputs prefilled with sentinels, so unwritten pad rows fail)."""
    from sageattention.sk1_backend.sk1_loader import SageLib
    lib = SageLib.get()
    kk, vv = (oracle.to_hnd(t, layout) for t in (k, v))
    B, H, N, D = kk.shape
    BH, n_pad = B * H, oracle.n_pad_for(N)
    dev = torch.device("cuda:0")
    k8 = torch.full((BH, n_pad, D), 0x5A, device=dev, dtype=torch.uint8)
    k8 = k8.view(torch.int8 if k_int8 else torch.float8_e4m3fn)
    v8t = torch.full((BH, D, n_pad), 0x5A, device=dev, dtype=torch.uint8).view(torch.float8_e4m3fn)
    sk, sv = (torch.full((BH, n_pad), float("nan"), device=dev) for _ in range(2))
    s = torch.full((BH,), float("nan"), device=dev)
    mean = torch.full((BH, D), float("nan"), device=dev)
    ws = torch.empty(lib.workspace_bytes(BH, N), device=dev, dtype=torch.uint8)
    lib.kv_prologue(kk.cuda(), vv.cuda(), k8, sk, v8t, sv, s, mean, ws, k_int8=k_int8,
                    smooth_k=True, fold=True, n_pad=n_pad)
    torch.cuda.synchronize()
    kr, vr = kk.reshape(BH, N, D), vv.reshape(BH, N, D)
    mu = oracle.kseq_mean(kr)
    r_k8, r_sk = oracle.quant_k(kr, n_pad, mean=mu, int8=k_int8)
    r_v8t, r_sv = oracle.quant_v(vr, n_pad)
    r_s, r_svp = oracle.fold_v_scale(r_sv)
    pairs = ((mean, mu), (k8, r_k8), (sk, r_sk), (v8t, r_v8t), (sv, r_svp), (s, r_s))
    return all(bytes_equal(g.cpu(), r) for g, r in pairs)


# (name, dtype, B, H, N, causal, layout, k_offset_std, outlier_frac, std), from BASELINE.json's
# configs: c1 (N=1024), c2 (N=8771, outlier keys), c3 (N=47520), c4 (bf16 N=16384), c5 (short and
# batched calls)
CASES = [
    ("c1", torch.float16, 1, 48, 1024, False, "HND", 2.0, 0.0, 1.0),
    ("c2n", torch.float16, 1, 48, 8771, False, "HND", 2.0, 0.001, 1.0),
    ("c2c", torch.float16, 1, 48, 8771, True, "HND", 2.0, 0.001, 1.0),
    ("c3n", torch.float16, 1, 48, 47520, False, "HND", 2.0, 0.0, 1.0),
    ("c3c", torch.float16, 1, 48, 47520, True, "HND", 2.0, 0.0, 1.0),
    ("c4", torch.bfloat16, 1, 48, 16384, True, "HND", 2.0, 0.001, 1.5),
    ("c5_288", torch.float16, 1, 48, 288, False, "HND", 0.0, 0.0, 1.0),
    ("c5_512", torch.float16, 1, 48, 512, False, "HND", 0.0, 0.0, 1.0),
    ("c5_4096", torch.float16, 1, 48, 4096, False, "HND", 0.0, 0.0, 1.0),
    ("c5_b8", torch.float16, 8, 24, 4096, False, "NHD", 0.0, 0.0, 1.0),
]


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--heads-cap", type=int, default=4,
                    help="heads per case (the N=47520 cases use half of it)")
    ap.add_argument("--only", default="", help="comma-separated case names")
    args = ap.parse_args()
    from sageattention import sageattn
    only = set(filter(None, args.only.split(",")))
    print("case dtype B H N causal layout | quantized bit-exact | cos rel_l1 (vs emulation) | "
          "emu_rel_rms gpu_rel_rms (vs exact) | seconds", flush=True)
    worst = {"cos": 1.0, "rel_l1": 0.0}
    all_exact = True
    for name, dt, B, H, N, causal, layout, off, outl, std in CASES:
        if only and name not in only:
            continue
        h = min(H, args.heads_cap if N < 32768 else max(1, args.heads_cap // 2))
        b = min(B, 2)
        t0 = time.time()
        q, k, v = make_qkv(b, h, N, seed=0, dtype=dt, layout=layout, std=std, k_offset_std=off,
                           outlier_frac=outl)
        out = sageattn(q.cuda(), k.cuda(), v.cuda(), tensor_layout=layout, is_causal=causal)
        torch.cuda.synchronize()
        out = out.cpu()
        emu = oracle.emulate_sageattn(q, k, v, tensor_layout=layout, is_causal=causal)["o"]
        ex = oracle.exact_attention(q, k, v, is_causal=causal, tensor_layout=layout)
        exact = quantized_bit_exact(k, v, layout, k_int8=(dt == torch.float16))
        all_exact = all_exact and exact
        c, r = cosine(out, emu), rel_l1(out, emu)
        worst["cos"] = min(worst["cos"], c)
        worst["rel_l1"] = max(worst["rel_l1"], r)
        print("%-8s %s %d %d %d %-5s %s | %s | %.6f %.3e | %.4f %.4f | %.0f" % (
            name, str(dt).split(".")[-1], b, h, N, causal, layout, "yes" if exact else "NO", c, r,
            rel_rms(emu, ex), rel_rms(out, ex), time.time() - t0), flush=True)
    print("worst: cos %.6f rel_l1 %.3e (bar: cos >= 0.999, rel_l1 <= 1e-2); quantized tensors "
          "bit-exact in every case: %s" % (worst["cos"], worst["rel_l1"], all_exact), flush=True)
    ok = worst["cos"] >= 0.999 and worst["rel_l1"] <= 1e-2 and all_exact
    return 0 if ok else 1


if __name__ == "__main__":
    sys.exit(main())
