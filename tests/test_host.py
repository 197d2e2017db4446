"""Host-side tests (CPU, no GPU): the C-ABI library exports, the stride rule, the envelope, and the
drop-in `sageattn`'s error behaviour."""
import ctypes
import inspect
import os
import re
import subprocess

import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "sage_mi355.h")


def _declared_symbols():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\**\s+\**(sage_\w+)\s*\(", text, flags=re.M)))


def test_header_declares_the_entry_points():
    syms = _declared_symbols()
    for s in ("sage_version", "sage_last_error", "sage_kv_prologue_workspace_bytes",
              "sage_kv_prologue", "sage_attn_fwd", "sage_attn_fwd_ex", "sage_attn_fwd_sk",
              "sage_kseq_mean", "sage_kv_prologue_noalloc",
              "sage_mfma_peak_probe", "sage_attn_kernel_choice",
              "sage_build_id", "sage_quant_q", "sage_mfma_layout_probe"):
        assert s in syms


def test_library_loads_and_exports_every_declared_symbol():
    from sageattention.sk1_backend import sk1_loader
    if not os.path.isfile(sk1_loader.LIB_PATH):
        pytest.skip("library not built (run __graft_entry__.build())")
    lib = ctypes.CDLL(sk1_loader.LIB_PATH)
    for s in _declared_symbols():
        assert hasattr(lib, s), s
    out = subprocess.run(["nm", "-D", "--defined-only", sk1_loader.LIB_PATH], capture_output=True,
                         text=True).stdout
    exported = set(re.findall(r" T (sage_\w+)", out))
    assert exported == set(_declared_symbols())


def test_kernel_choice_by_grid_fill():
    # The automatic main-loop choice on 256 CUs (no device query when the CU count is given).
    # head_dim 64: the key split when not causal with at most 6 of its 64-query blocks per CU.
    # Causal: the 256-query ping-pong from 4 of its blocks per CU (1024 blocks). Non-causal: whole
    # rounds of blocks (three 128-query blocks or one 256-query block per CU) at the measured
    # per-CU throughputs 1.00 / 1.52 / 1.69 and 1.75; the ping-pong when >= 3 % sooner.
    from sageattention.sk1_backend import sk1_loader
    if not os.path.isfile(sk1_loader.LIB_PATH):
        pytest.skip("library not built")
    L = sk1_loader.SageLib.get()
    Q256, PIPE, SPLIT = 2, 3, 4
    cases = [
        # (B, H, N, D, causal, expected)
        (1, 48, 47520, 128, True, Q256),    # the headline: 8928 blocks of 256 queries
        (1, 48, 47520, 64, True, PIPE),     # head_dim 64 causal: always the pipelined kernel
        (1, 10, 4096, 64, True, PIPE),
        (1, 10, 4096, 64, False, SPLIT),    # 640 blocks of 64 queries <= 6 per CU: key split
        (1, 24, 4096, 64, False, SPLIT),    # 1536 blocks: the limit
        (1, 25, 4096, 64, False, PIPE),     # 1600 blocks
        (1, 24, 4097, 64, False, PIPE),     # 1560 blocks
        (1, 48, 4096, 64, False, PIPE),
        (1, 30, 17550, 64, False, PIPE),    # CogVideoX-like: 32 per CU
        (2, 1, 1, 64, False, SPLIT),
        (1, 48, 4096, 128, True, PIPE),     # 768 blocks < 1024
        (1, 8, 32768, 128, True, Q256),     # exactly 1024 blocks
        (1, 8, 32512, 128, True, PIPE),     # 1016 blocks
        (1, 48, 8771, 128, True, PIPE),     # 1680 blocks, but the last tile pads 189 of 256 rows:
                                            # 2*189/8771 = 4.3 % more causal work, 1.4 % at 128
        (1, 48, 47520, 128, True, Q256),    # pads 96 rows: 0.4 % against 0.1 %
        # non-causal, in units of one 128-query block alone on a CU:
        (1, 48, 1024, 128, False, Q256),    # 384 blocks: two on half the CUs, 2/1.52 = 1.32;
                                            # 192 blocks of 256 in one round: 2/1.75 = 1.14
        (1, 48, 512, 128, False, PIPE),     # 192 blocks, one per CU: 1.00 against 1.14
        (1, 48, 2048, 128, False, PIPE),    # one round of three, 3/1.69 = 1.78 against 2.29
        (1, 48, 8771, 128, False, PIPE),    # 4 rounds of three + 1 block: 8.10 against 7 x 1.14
                                            # = 8.00, not 3 % sooner
        (1, 48, 47520, 128, False, Q256),   # 23 x 1.78 + 1 = 41.8 against 35 x 1.14 = 40.0
        (1, 8, 8192, 128, False, Q256),     # 512 blocks: 1.32 against one round, 1.14
        (1, 8, 12288, 128, False, PIPE),    # one round of three: 1.78 against 2.29
    ]
    for B, H, N, D, causal, want in cases:
        assert L.kernel_choice(B, H, N, D, causal, cus=256) == want, (B, H, N, D, causal)
    with pytest.raises(ValueError, match="shape"):
        L.kernel_choice(0, 48, 1024, 128, False, cus=256)
    with pytest.raises(ValueError, match="head_dim"):
        L.kernel_choice(1, 48, 1024, 96, False, cus=256)


def test_library_host_calls_without_a_gpu():
    # Calls that touch no device: the version, the workspace size, and argument refusals (which
    # are checked before any launch).
    from sageattention.sk1_backend import sk1_loader
    if not os.path.isfile(sk1_loader.LIB_PATH):
        pytest.skip("library not built")
    L = sk1_loader.SageLib.get()
    assert L.version == 200
    assert L.workspace_bytes(48, 47520) > 48 * 128 * 8
    assert L.workspace_bytes(1, 1) > 0
    i64 = ctypes.c_int64
    rc = L.lib.sage_attn_fwd(0, 1, 1, None, 8, 8, 8, None, None, None, None, None, 8, 8, 8,
                             1, 1, 0, 64, ctypes.c_float(0.1), None)
    assert rc == 1 and b"n_lt_1" in L.lib.sage_last_error()
    rc = L.lib.sage_kv_prologue(1, 1, 1, 0, 1, None, 8, 8, 8, None, 8, 8, 8, 1, 1, 10, 64, 128,
                                *([None] * 9), 0, None)
    assert rc == 1 and b"bf16_int8" in L.lib.sage_last_error()
    rc = L.lib.sage_kv_prologue(0, 1, 1, 0, 1, ctypes.c_void_p(16), 8, 8, 4, ctypes.c_void_p(16),
                                8, 8, 8, 1, 1, 10, 64, 128, *([None] * 9), 0, None)
    assert rc == 1 and b"stride_align" in L.lib.sage_last_error()
    rc = L.lib.sage_attn_fwd(0, 1, 0, ctypes.c_void_p(16), 8, 8, 8, None, None, None, None,
                             ctypes.c_void_p(16), 8, 8, 8, 1, 1, 100, 96, ctypes.c_float(0.1), None)
    assert rc == 1 and b"n_pad" in L.lib.sage_last_error()
    p16 = ctypes.c_void_p(16)
    def ex(causal=0, H=1, N=100, H_kv=1, N_kv=100, N_kv_pad=128, kernel=0, lse=None, D=128):
        return L.lib.sage_attn_fwd_ex(0, 1, causal, p16, 12800, 12800, 128, p16, p16, p16, p16,
                                      p16, 12800, 12800, 128, 1, H, N, H_kv, N_kv, N_kv_pad, D,
                                      ctypes.c_float(0.1), kernel, lse, None, None, None)
    assert ex(kernel=7) == 1 and b"kernel" in L.lib.sage_last_error()
    assert ex(lse=ctypes.c_void_p(18)) == 1
    assert b"lse must be 4-byte aligned" in L.lib.sage_last_error()
    # grouped K/V heads: H must be a multiple of H_kv; causal needs N == N_kv
    assert ex(H=6, H_kv=4) == 1 and b"heads" in L.lib.sage_last_error()
    assert ex(H=1, H_kv=0) == 1 and b"heads" in L.lib.sage_last_error()
    assert ex(causal=1, N_kv=99) == 1 and b"seq_len" in L.lib.sage_last_error()
    assert ex(N_kv=200, N_kv_pad=192) == 1 and b"n_pad" in L.lib.sage_last_error()
    assert ex(N_kv=0, N_kv_pad=64) == 1 and b"n_lt_1" in L.lib.sage_last_error()
    # head_dim 64 or 128; 64 only on the 128-query kernel
    assert ex(D=96) == 1 and b"head_dim" in L.lib.sage_last_error()
    assert ex(D=64, kernel=2) == 1 and b"kernel" in L.lib.sage_last_error()
    # the key split: non-causal head_dim 64 only, and its 64-query grid within HIP's limit
    assert ex(kernel=4) == 1 and b"key-split" in L.lib.sage_last_error()
    assert ex(D=64, causal=1, kernel=4) == 1 and b"key-split" in L.lib.sage_last_error()
    assert ex(D=64, kernel=4, H=4194305, N=200, N_kv=100) == 1
    assert b"the key-split main loop needs 16777220 blocks" in L.lib.sage_last_error()
    rc = L.lib.sage_quant_q(0, 1, p16, 12800, 12800, 128, 1, 1, 100, 32, ctypes.c_float(0.1),
                            p16, p16, p16, None)
    assert rc == 1 and b"head_dim" in L.lib.sage_last_error()
    # the workspace size depends on B*H and N only: with N_pad = 256 > ceil(N/64)*64 the refusal
    # names the same size as workspace_bytes(B*H, N). (No call here passes every check: on a host
    # with a GPU such a call would launch kernels on these made-up addresses.)
    need = L.workspace_bytes(1, 64)
    assert need == L.workspace_bytes(1, 33)
    rc = L.lib.sage_kv_prologue(0, 1, 1, 0, 1, p16, 64 * 128, 64 * 128, 128, p16, 64 * 128,
                                64 * 128, 128, 1, 1, 64, 256, 128, p16, p16, p16, p16, None,
                                None, p16, None, ctypes.c_void_p(256), need - 8, None)
    assert rc == 1 and b"workspace" in L.lib.sage_last_error()
    assert b"need %d bytes" % need in L.lib.sage_last_error()
    # the no-allocation prologue refuses, before touching a GPU, a call whose workspace exceeds
    # its static scratch (4 MiB): here 4096 planes need 8 MiB
    assert L.workspace_bytes(4096, 64) > (4 << 20) >= L.workspace_bytes(24, 9000)
    rc = L.lib.sage_kv_prologue_noalloc(0, 1, 1, 0, 1, p16, 64 * 128, 64 * 128, 128, p16,
                                        64 * 128, 64 * 128, 128, 1, 4096, 64, 64, 128, p16, p16,
                                        p16, p16, None, None, p16, None, None)
    assert rc == 1 and b"scratch" in L.lib.sage_last_error()
    # the MFMA probe's bounds
    assert L.lib.sage_mfma_peak_probe(1, 0, 10, None, None) == 1
    assert b"blocks" in L.lib.sage_last_error()
    assert L.lib.sage_mfma_peak_probe(0, 8, 0, None, None) == 1
    assert b"iters" in L.lib.sage_last_error()
    assert L.lib.sage_mfma_peak_probe(0, 8, 8, ctypes.c_void_p(12), None) == 1
    assert b"aligned" in L.lib.sage_last_error()
    # B*H beyond 65535 is a valid shape (the grids are 1-D); HIP's 2^32-1 threads per launch bound
    # each grid: 128-query blocks of 256 threads and 256-query blocks of 512 (main loop), 64-row
    # blocks of 64 threads (Q quantizer), one 256-thread block per plane at B*H >= 2048 (prologue)
    def fwd(H, N):
        return L.lib.sage_attn_fwd(0, 1, 0, p16, 8, 8, 8, None, None, None, None, p16, 8, 8, 8,
                                   1, H, N, (N + 63) // 64 * 64, ctypes.c_float(0.1), None)
    assert fwd(70000, 100) == 1 and b"NULL" in L.lib.sage_last_error()
    assert fwd((1 << 17) - 1, 16384) == 1 and b"NULL" in L.lib.sage_last_error()
    assert fwd(1 << 17, 16384) == 1 and b"grid" in L.lib.sage_last_error()
    assert fwd((1 << 17) - 1, 16385) == 1 and b"grid" in L.lib.sage_last_error()
    rc = L.lib.sage_attn_fwd(0, 1, 0, p16, 8, 8, 8, None, None, None, None, p16, 8, 8, 8,
                             1 << 20, 1 << 12, 1 << 10, 1 << 10, ctypes.c_float(0.1), None)
    assert rc == 1 and b"grid" in L.lib.sage_last_error()
    def qq(H, N):
        return L.lib.sage_quant_q(0, 1, p16, 8, 8, 8, 1, H, N, 128, ctypes.c_float(0.1), None,
                                  None, None, None)
    assert qq((1 << 20) - 1, 2048) == 1 and b"NULL" in L.lib.sage_last_error()
    assert qq(1 << 20, 2048) == 1 and b"grid" in L.lib.sage_last_error()
    def pro(H):
        return L.lib.sage_kv_prologue(0, 1, 1, 0, 1, p16, 8, 8, 8, p16, 8, 8, 8, 1, H, 64, 64,
                                      128, *([None] * 9), 0, None)
    assert pro((1 << 24) - 1) == 1 and b"NULL" in L.lib.sage_last_error()
    assert pro(1 << 24) == 1 and b"grid" in L.lib.sage_last_error()
    # the main loop on SK / SV' and the mean alone refuse like the others
    def sk(**kw):
        a = dict(dtype=0, qk_int8=1, causal=0, D=128, H_kv=1, N_kv=100, sk=p16)
        a.update(kw)
        return L.lib.sage_attn_fwd_sk(a["dtype"], a["qk_int8"], a["causal"], p16, 12800, 12800,
                                      128, p16, a["sk"], p16, p16, None, p16, p16, 12800, 12800,
                                      128, 1, 1, 100, a["H_kv"], a["N_kv"], 128, a["D"],
                                      ctypes.c_float(0.1), None, None, None)
    assert sk(dtype=1) == 1 and b"bf16_int8" in L.lib.sage_last_error()
    assert sk(D=96) == 1 and b"head_dim" in L.lib.sage_last_error()
    assert sk(causal=1, N_kv=99) == 1 and b"seq_len" in L.lib.sage_last_error()
    assert sk(sk=ctypes.c_void_p(20)) == 1 and b"ptr_align" in L.lib.sage_last_error()
    assert sk(sk=None) == 1 and b"NULL" in L.lib.sage_last_error()
    rc = L.lib.sage_kseq_mean(0, p16, 12800, 12800, 128, 1, 1, 100, 96, p16, p16, 1 << 20, None)
    assert rc == 1 and b"mean_head_dim" in L.lib.sage_last_error()
    rc = L.lib.sage_kseq_mean(0, p16, 12800, 12800, 128, 1, 1, 100, 128, p16, p16, 8, None)
    assert rc == 1 and b"workspace" in L.lib.sage_last_error()
    # smooth_v needs somewhere to put V's mean
    rc = L.lib.sage_kv_prologue(0, 1, 1, 1, 1, p16, 12800, 12800, 128, p16, 12800, 12800, 128,
                                1, 1, 100, 128, 128, p16, p16, p16, p16, None, None, p16, None,
                                p16, 1 << 20, None)
    assert rc == 1 and b"vmean" in L.lib.sage_last_error()


def test_library_shares_torch_hip_runtime():
    # the library's libamdhip64 dependency resolves to the image torch already loaded, so torch's
    # stream handles are valid for its launches
    from sageattention.sk1_backend import sk1_loader
    if not os.path.isfile(sk1_loader.LIB_PATH):
        pytest.skip("library not built")
    L = sk1_loader.SageLib.get()
    assert L.hip_runtime and len(L.hip_runtime) == 1, L.hip_runtime
    assert L.same_as_torch is True


def test_strided_view_reason_rule():
    from sageattention.sk1_backend.sk1_loader import strided_view_reason as r
    t = torch.empty(2, 4, 100, 128, dtype=torch.float16)
    assert r(t) is None
    assert r(t.transpose(1, 2).contiguous().transpose(1, 2)) is None        # physically NHD
    assert r(t[..., :64]) is None
    assert r(t[:, :, :, 1:65]) == "ptr_align"
    assert r(t.transpose(2, 3)) == "stride_last"
    assert r(t[0]) == "rank"
    assert r(t.expand(2, 4, 100, 128).as_strided((2, 4, 100, 128), (0, 12800, 128, 1))) == "stride_nonpos"
    assert r(torch.empty(1, 1, 4, 136, dtype=torch.float16)[..., :128]) is None
    assert r(torch.empty(1, 1, 4, 132, dtype=torch.float16)[..., :128]) == "stride_align"
    over = torch.empty(4096, dtype=torch.float16).as_strided((1, 2, 10, 128), (2048, 64, 128, 1))
    assert r(over) == "stride_overlap"
    # fused QKV split: row stride 3*H*D, B=1 via unsqueeze (size-1 dims are ignored)
    qkv = torch.empty(100, 3 * 4 * 128, dtype=torch.float16)
    q = qkv.split(4 * 128, dim=-1)[1].view(100, 4, 128).transpose(0, 1).unsqueeze(0)
    assert r(q) is None
    # strides beyond int32 are served (every address is formed in 64 bits): no stride_int32
    big = torch.empty(1, dtype=torch.float16, device="meta").as_strided(
        (2, 1, 4, 128), (2 ** 31 + 1024, 512, 128, 1))
    assert r(big) is None


def test_refusal_vocabularies():
    from sageattention.sk1_backend.hip_prologue import REFUSALS
    from sageattention.sk1_backend.sk1_loader import STRIDED_REFUSALS
    assert "stride_int32" not in STRIDED_REFUSALS
    for p in ("k_", "v_", "mean_"):
        for r in STRIDED_REFUSALS:
            assert p + r in REFUSALS
    assert len(set(REFUSALS)) == len(REFUSALS)


def test_envelope_reasons_on_cpu_tensors():
    from sageattention.sk1_backend import _envelope_ok
    q = torch.empty(1, 2, 10, 128, dtype=torch.float16)
    args = dict(tensor_layout="HND", is_causal=False, sm_scale=None, return_lse=False,
                smooth_k=True, smooth_v=False, attn_mask=None)
    assert _envelope_ok(q, q, q, **dict(args, tensor_layout="BHND")) == "layout"
    # return_lse is served here (the reference's SK1 path refuses it): CPU tensors then fail
    # on the device check, not on return_lse
    assert _envelope_ok(q, q, q, **dict(args, return_lse=True)) == "device"
    # smooth_v is served too (the reference's SK1 envelope refuses it)
    assert _envelope_ok(q, q, q, **dict(args, smooth_v=True)) == "device"
    assert _envelope_ok(q, q, q, **dict(args, attn_mask=torch.ones(1))) == "attn_mask"
    assert _envelope_ok(q, q, q, **args) == "device"


def test_sageattn_signature_and_refusals():
    from sageattention import sageattn
    params = list(inspect.signature(sageattn).parameters)
    assert params[:7] == ["q", "k", "v", "tensor_layout", "is_causal", "sm_scale", "return_lse"]
    assert "attn_mask" not in params                   # ComfyUI probes for its absence
    q = torch.empty(1, 2, 10, 128, dtype=torch.float16)
    with pytest.raises(NotImplementedError):
        sageattn(q, q, q, attn_mask=torch.ones(1))
    with pytest.raises(ValueError, match="device"):
        sageattn(q, q, q)
    with pytest.raises(TypeError):
        sageattn(q, q, q, no_such_kwarg=1)


def test_try_sk1_t1_returns_reasons():
    from sageattention.sk1_backend import try_sk1_t1
    q = torch.empty(1, 2, 10, 128, dtype=torch.float16)
    assert try_sk1_t1(q, q, q) == (None, "device")
    assert try_sk1_t1(q, q, q, return_lse=True) == (None, "device")


def test_arch_gate_is_monkeypatchable(monkeypatch):
    import sageattention.sk1_backend as sk1
    monkeypatch.setattr(sk1, "device_arch", lambda device=None: "gfx942")
    assert not sk1.arch_supported(None)
    monkeypatch.setattr(sk1, "device_arch", lambda device=None: "gfx950")
    assert sk1.arch_supported(None)


def test_product_path_has_no_oracle_or_cpu_fallback():
    # The shipped package never imports the test oracle, and has no torch-only attention path.
    pkg = os.path.join(ROOT, "sageattention-rdna4_amd", "sageattention")
    for dirpath, _, files in os.walk(pkg):
        for f in files:
            if f.endswith(".py"):
                src = open(os.path.join(dirpath, f)).read()
                assert "oracle" not in src, f
                assert "scaled_dot_product_attention" not in src, f


def test_library_build_id_is_this_trees():
    # the library reports the hash of the sources and flags it was compiled from; the loaded one
    # must be this tree's (build_lib.source_hash), else it is stale
    import build_lib
    from sageattention.sk1_backend.sk1_loader import SageLib
    bid = SageLib.get().build_id
    assert len(bid) == 16 and bid == build_lib.source_hash()
