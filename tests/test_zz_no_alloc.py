"""`sage_kv_prologue_noalloc` (the prologue on the library's static per-GPU scratch) against
`sage_kv_prologue` with a caller-allocated workspace (GPU).

Two calls in a row through the C ABI, the second on a smaller input, each compared bit for bit
with the allocating entry point on the same inputs: every output (K8, SK, V8T, SV', S, MEAN, VMEAN,
KCONST). The second call's scratch still holds the first call's partials, so a partial it failed to
write would show up as a mismatch.
"""
import pytest
import torch

from sage_testutil import bytes_equal, have_gfx950, make_qkv, mismatch_report

pytestmark = [pytest.mark.gpu,
              pytest.mark.skipif(not have_gfx950(), reason="needs a gfx950 GPU")]

SCRATCH_BYTES = 4 << 20


def _outputs(BH, n_pad, D, k_int8, dev):
    def fill(shape, dtype):
        if dtype in (torch.int8, torch.float8_e4m3fn):
            return torch.full(shape, 0x5A, device=dev, dtype=torch.uint8).view(dtype)
        return torch.full(shape, float("nan"), device=dev, dtype=dtype)
    return dict(k8=fill((BH, n_pad, D), torch.int8 if k_int8 else torch.float8_e4m3fn),
                sk=fill((BH, n_pad), torch.float32), v8t=fill((BH, D, n_pad), torch.float8_e4m3fn),
                sv=fill((BH, n_pad), torch.float32), s=fill((BH,), torch.float32),
                mean=fill((BH, D), torch.float32), vmean=fill((BH, D), torch.float32),
                kconst=fill((BH, n_pad // 64, 2, 64), torch.float32))


def _both(lib, k, v, *, k_int8, smooth_k, smooth_v):
    B, H, N, D = k.shape
    BH, n_pad = B * H, (N + 63) // 64 * 64
    assert lib.workspace_bytes(BH, N) <= SCRATCH_BYTES
    ref = _outputs(BH, n_pad, D, k_int8, k.device)
    ws = torch.empty(lib.workspace_bytes(BH, N), device=k.device, dtype=torch.uint8)
    lib.kv_prologue(k, v, ref["k8"], ref["sk"], ref["v8t"], ref["sv"], ref["s"], ref["mean"], ws,
                    k_int8=k_int8, smooth_k=smooth_k, fold=True, n_pad=n_pad,
                    kconst=ref["kconst"], smooth_v=smooth_v, vmean=ref["vmean"])
    got = _outputs(BH, n_pad, D, k_int8, k.device)
    lib.kv_prologue_noalloc(k, v, got["k8"], got["sk"], got["v8t"], got["sv"], got["s"],
                            got["mean"], k_int8=k_int8, smooth_k=smooth_k, fold=True, n_pad=n_pad,
                            kconst=got["kconst"], smooth_v=smooth_v, vmean=got["vmean"])
    torch.cuda.synchronize()
    for name in ref:
        a, b = got[name].cpu(), ref[name].cpu()
        assert bytes_equal(a, b), mismatch_report(a, b, name)


@pytest.mark.parametrize("dtype,k_int8", [(torch.float16, True), (torch.bfloat16, False)])
def test_noalloc_prologue_equals_the_workspace_entry_twice(dtype, k_int8):
    from sageattention.sk1_backend.sk1_loader import SageLib
    lib = SageLib.get()
    # first call: 24 planes of 9000 keys with smooth_k and smooth_v (both partial regions in use)
    print("noalloc call 1", dtype, flush=True)
    _, k, v = make_qkv(2, 12, 9000, seed=1, dtype=dtype, k_offset_std=2.0, outlier_frac=0.001,
                       v_offset_std=1.0)
    v[1, 3, 17] = 4000.0
    _both(lib, k.cuda(), v.cuda(), k_int8=k_int8, smooth_k=True, smooth_v=True)
    # second call, smaller: 3 planes of 700 keys, smooth_k only, NHD-strided views
    print("noalloc call 2", dtype, flush=True)
    _, k, v = make_qkv(1, 3, 700, seed=2, dtype=dtype, k_offset_std=2.0, layout="NHD")
    kd, vd = (t.cuda().transpose(1, 2) for t in (k, v))
    _both(lib, kd, vd, k_int8=k_int8, smooth_k=True, smooth_v=False)


def test_noalloc_prologue_refuses_beyond_the_scratch():
    from sageattention.sk1_backend.sk1_loader import SageLib
    lib = SageLib.get()
    B, H, N = 1, 4096, 64
    assert lib.workspace_bytes(B * H, N) > SCRATCH_BYTES
    k = torch.empty(B, H, N, 128, device="cuda", dtype=torch.float16)
    out = _outputs(B * H, 64, 128, True, k.device)
    with pytest.raises(ValueError, match="scratch"):
        lib.kv_prologue_noalloc(k, k, out["k8"], out["sk"], out["v8t"], out["sv"], out["s"],
                                out["mean"], k_int8=True, smooth_k=True, fold=True, n_pad=64)
