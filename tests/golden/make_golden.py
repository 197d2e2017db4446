"""Write the golden fixtures under tests/golden/ (run from the repository root).

    python tests/golden/make_golden.py

The reference holds no golden vectors for this path (its tests are relational and tolerance
checks), so these fixtures freeze the CPU oracle's outputs on small, seeded inputs that exercise
the scheme's corner cases: ragged tails (N not a multiple of 64), a single token, the smooth_k
mean, outlier keys, an all-zero key row and an all-zero value row (the 1e-12 scale floor), and
value rows above 448 (the S > 1 fold). The oracle is pinned independently by tests/test_oracle.py
(closed forms, an independent e4m3 encoder, exact sums, brute force); the fixtures then catch any
drift of the oracle itself (tests/test_golden.py re-derives them on the CPU) and give the GPU tests
stored expected bits.

Each fixture is an .npz of plain arrays (no pickles): inputs as raw 16-bit patterns, every
quantized tensor and scale, and the emulated output's 16-bit patterns.
"""
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.abspath(os.path.join(HERE, "..", "..")))
sys.path.insert(0, os.path.abspath(os.path.join(HERE, "..")))
import oracle  # noqa: E402
from sage_testutil import make_qkv  # noqa: E402

CASES = {
    # name: (dtype, B, H, N, causal, smooth_k, layout, std, k_offset, outliers, seed
    #        [, H_kv, N_kv[, smooth_v, v_offset[, head_dim]]]])
    "fp16_n77_causal": (torch.float16, 1, 1, 77, True, True, "HND", 1.0, 2.0, 0.03, 11),
    "fp16_n1_noncausal": (torch.float16, 1, 2, 1, False, True, "HND", 1.0, 2.0, 0.0, 12),
    "fp16_n70_nhd_nosmooth": (torch.float16, 2, 1, 70, False, False, "NHD", 1.0, 0.0, 0.0, 13),
    "bf16_n67_causal": (torch.bfloat16, 1, 1, 67, True, True, "HND", 1.5, 2.0, 0.02, 14),
    # grouped K/V heads with a longer key sequence; one shared K/V head with a shorter one
    "fp16_gqa_h4kv2_n70_kv130": (torch.float16, 1, 4, 70, False, True, "HND", 1.0, 2.0, 0.02, 15,
                                 2, 130),
    "bf16_mqa_nhd_n100_kv37": (torch.bfloat16, 2, 3, 100, False, True, "NHD", 1.0, 1.0, 0.0, 16,
                               1, 37),
    # smooth_v on V with per-channel offsets
    "fp16_smoothv_n100_causal": (torch.float16, 1, 2, 100, True, True, "HND", 1.0, 2.0, 0.0, 17,
                                 2, 100, True, 4.0),
    "bf16_smoothv_gqa_n80_kv150": (torch.bfloat16, 1, 4, 80, False, False, "HND", 1.0, 0.0, 0.0,
                                   18, 2, 150, True, 3.0),
    # head_dim 64
    "fp16_d64_n90_causal": (torch.float16, 1, 2, 90, True, True, "HND", 1.0, 2.0, 0.03, 19,
                            2, 90, False, 0.0, 64),
    "bf16_d64_gqa_nhd_n50_kv77_smoothv": (torch.bfloat16, 1, 4, 50, False, True, "NHD", 1.0, 1.5,
                                          0.0, 20, 2, 77, True, 2.0, 64),
}


def bits(t):
    """Raw bit patterns of a tensor as a numpy array (16-bit floats -> uint16, e4m3 -> uint8)."""
    t = t.contiguous()
    if t.dtype in (torch.float16, torch.bfloat16):
        return t.view(torch.int16).numpy().view(np.uint16)
    if t.dtype == torch.float8_e4m3fn:
        return t.view(torch.uint8).numpy()
    return t.numpy()


def corner_rows(q, k, v, layout):
    """Plant the corner cases into plane 0 (in the logical HND view)."""
    kk, vv = (oracle.to_hnd(t, layout) for t in (k, v))
    N = kk.shape[2]
    if N >= 3:
        kk[0, 0, 1] = 0          # an all-zero key row: K's scale hits the floor when not smoothed
        vv[0, 0, 2] = 0          # an all-zero value row: V's scale hits the floor
        vv[0, 0, 0, :7] = torch.tensor([900., -613., 450., 448., 449., -2000., 7.], dtype=v.dtype)
    return q, k, v


def make(name):
    dtype, B, H, N, causal, smooth_k, layout, std, off, outl, seed = CASES[name][:11]
    H_kv, N_kv = CASES[name][11:13] or (H, N)
    smooth_v, v_off = CASES[name][13:15] or (False, 0.0)
    D = CASES[name][15] if len(CASES[name]) > 15 else 128
    q, k, v = make_qkv(B, H, N, seed=seed, dtype=dtype, layout=layout, std=std, k_offset_std=off,
                       outlier_frac=outl, h_kv=H_kv, n_kv=N_kv, v_offset_std=v_off, d=D)
    q, k, v = corner_rows(q, k, v, layout)
    r = oracle.emulate_sageattn(q, k, v, tensor_layout=layout, is_causal=causal, smooth_k=smooth_k,
                                smooth_v=smooth_v)
    arr = dict(
        # B, H, N, causal, smooth_k, NHD, bf16, H_kv, N_kv, smooth_v, head_dim
        meta=np.array([B, H, N, int(causal), int(smooth_k), int(layout == "NHD"),
                       int(dtype == torch.bfloat16), H_kv, N_kv, int(smooth_v), D], dtype=np.int64),
        sm_scale=np.array([r["sm_scale"]], dtype=np.float32),
        q=bits(q), k=bits(k), v=bits(v),
        k8=bits(r["k8"]) if r["k8"].dtype != torch.int8 else r["k8"].numpy(),
        sk=r["sk"].numpy(), v8t=bits(r["v8t"]), sv=r["sv"].numpy(), s=r["s"].numpy(),
        svp=r["svp"].numpy(), q8=bits(r["q8"]) if r["q8"].dtype != torch.int8 else r["q8"].numpy(),
        sq=r["sq"].numpy(), c_q=r["c_q"].numpy(), o=bits(r["o"]), lse=r["lse"].numpy(),
    )
    if r["mean"] is not None:
        arr["mean"] = r["mean"].numpy()
    if r["vmean"] is not None:
        arr["vmean"] = r["vmean"].numpy()
    return arr


def main():
    for name in CASES:
        path = os.path.join(HERE, name + ".npz")
        np.savez_compressed(path, **make(name))
        print("wrote", os.path.relpath(path), os.path.getsize(path), "bytes")


if __name__ == "__main__":
    main()
