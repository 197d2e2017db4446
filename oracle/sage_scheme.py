"""The SK1 quantization scheme and attention loop, restated on the CPU in PyTorch fp32.

TEST INFRASTRUCTURE ONLY (see the package docstring): the checker for the gfx950 kernels, never the
product.

Conventions:
* RN(x) is one IEEE fp32 round-to-nearest-even operation. Every fp32 operation below is a single
  torch CPU op on fp32 tensors, so each is one correctly rounded IEEE operation. No fused
  multiply-add and no reassociation are used anywhere in the quantizers.
* `torch.round` is round-half-to-even, the rule of `rintf` / `v_rndne_f32`.
* `.to(torch.float8_e4m3fn)` is the OCP e4m3fn cast with round-to-nearest-even, the rule of the
  hardware `v_cvt_pk_fp8_f32`. Every value cast here is already bounded by 448 in magnitude (up to
  one fp32 rounding), so the cast's out-of-range behaviour is never reached.
* Shapes are per (b, h) plane, flattened to `BH = B*H` in the leading axis: Q/K/V are (BH, N, D).

Reference files (paths relative to the reference repository root):
* `kernels/hip/h34_prologue.hip` -- the K/V prologue and the smooth_k mean;
* `kernels/hip/sk1_t6i.hip` -- int8 Q.K main loop (fp16 inputs);
* `kernels/hip/sk1_t4a1s.hip`, `kernels/hip/sk1_t4a1sb.hip` -- fp8 Q.K main loop (bf16 inputs);
* `sageattention/sk1_backend/__init__.py` -- the per-(b,h) V-scale fold and the routing;
* `sageattention/sk1_backend/hip_prologue.py` -- `n_pad_for`, the scale floor;
* `sageattention/sk1_backend/quant_triton.py` -- the reference's fp32 sequence mean of its own
  smooth_v path (`vseq_mean_fp32_chunked`).

Parity status: every function here is pinned by `tests/test_oracle.py` and the golden fixtures.
For `vseq_mean_fp32_chunked` the pin covers everything the reference fixes (fp32 accumulation of
16-row group sums in row order per 1024-row chunk, chunk partials in chunk order, one fp32
division), on data where that accumulation must round; the order inside one 16-row Triton
`tl.sum` is not fixed by the reference and is taken as a pairwise tree.
"""
import math

import torch

#: Key-tile width of the reference main loop and the padding granule of every quantized tensor
#: (`kernels/hip/sk1_t6i.hip:24`, `sageattention/sk1_backend/hip_prologue.py:66`).
BN = 64
#: The int8/fp8 scale floor, fp32(1e-12) (`hip_prologue.py:188`, `h34_prologue.hip:147`).
FLOOR = torch.tensor(1e-12, dtype=torch.float32)
#: fp32(log2(e)) (`kernels/hip/sk1_t6i.hip:29`).
LOG2E = torch.tensor(1.4426950408889634, dtype=torch.float32)
#: e4m3 maximum and the P fold multiplier (`kernels/hip/sk1_t6i.hip:27`).
P_SCALE = torch.tensor(448.0, dtype=torch.float32)
#: int8 quantization range (`kernels/hip/sk1_t6i.hip:28`).
I8_MAX = torch.tensor(127.0, dtype=torch.float32)

F8 = torch.float8_e4m3fn


def n_pad_for(N):
    """`N_pad = ceil(N/64)*64` (`sageattention/sk1_backend/hip_prologue.py:93-95`)."""
    return ((int(N) + BN - 1) // BN) * BN


def to_hnd(x, tensor_layout):
    """The logical (B, H, N, D) reading of a caller tensor (`sk1_backend/__init__.py:1035-1038`)."""
    return x.transpose(1, 2) if tensor_layout == "NHD" else x


def kseq_mean(k):
    """smooth_k's sequence-axis mean (`kernels/hip/h34_prologue.hip:259-282`).

    `mu[bh, d] = fp32( (sum_n fp64(k[bh, n, d])) / fp64(N) )`: every element is widened exactly to
    fp64, summed in fp64, divided once in fp64 and rounded once to fp32. The fp64 sum is exact (so
    independent of order) whenever every partial sum is representable, which holds for fp16 inputs
    of magnitude below 2^10 at N < 2^19; the reference kernel's result is then the same bits.
    `k`: (BH, N, D) fp16/bf16. Returns (BH, D) fp32.
    """
    N = k.shape[1]
    s = k.to(torch.float64).sum(dim=1)
    return (s / float(N)).to(torch.float32)


def vseq_mean_fp32_chunked(x, chunk=1024, group=16):
    """The sequence mean as the reference's own smooth_v path computes it: `kseq_mean_fp8`
    (`sageattention/sk1_backend/quant_triton.py:303-373`), which its Triton prologue subtracts from V
    under `SUB_VMEAN` (`quant_triton.py:714-719`).

    Stage 1 (`_kseq_partial_sum`, `:303-331`): per chunk of `chunk` rows an fp32 accumulator, zeroed,
    receives `group`-row sums in row order (`acc += tl.sum(x[16 rows], axis=0)`, rows past N
    read as 0). Stage 2 (`_kseq_finalize_mean`, `:334-343`): the chunk partials summed in chunk order
    in fp32, then one fp32 division by N. The order inside one 16-row `tl.sum` is Triton's
    reduction tree, which the reference does not fix; it is taken here as a balanced pairwise tree
    (rows 0+1, 2+3, ..., then pairs of pairs). Where each group's sum is exact in fp32 (every
    order then agrees), this is the reference's function bit for bit; the tests pin it there
    against an exact rational simulation, with the rounding the fp32 accumulation forces.
    `x`: (BH, N, D) fp16/bf16. Returns (BH, D) fp32.
    """
    BH, N, D = x.shape
    xf = x.to(torch.float32)
    n_ch = (N + chunk - 1) // chunk
    parts = []
    for c in range(n_ch):
        acc = torch.zeros(BH, D, dtype=torch.float32)
        for r in range(c * chunk, (c + 1) * chunk, group):
            g = torch.zeros(BH, group, D, dtype=torch.float32)
            hi = min(r + group, N)
            if hi > r:
                g[:, : hi - r] = xf[:, r:hi]
            while g.shape[1] > 1:
                g = g[:, 0::2] + g[:, 1::2]
            acc = acc + g[:, 0]
        parts.append(acc)
    tot = torch.zeros(BH, D, dtype=torch.float32)
    for p_ in parts:
        tot = tot + p_
    return tot / torch.tensor(float(N), dtype=torch.float32)


def _pad_rows(x, n_pad):
    BH, N, D = x.shape
    out = torch.zeros(BH, n_pad, D, dtype=torch.float32)
    out[:, :N] = x.to(torch.float32)
    return out


def quant_k(k, n_pad, mean=None, int8=True):
    """K per-token quantization (`kernels/hip/h34_prologue.hip:116-165`).

    * `kc = RN(fp32(k) - mu)` when a mean is given, else `fp32(k)`; pad rows (n >= N) are 0;
    * `kmax = max_d |kc|`;
    * int8 (fp16 inputs): `sk = max(RN(kmax / 127), FLOOR)`,
      `K8 = clamp(rne(RN(kc / sk)), -128, 127)` -- a correctly rounded DIVISION
      (`h34_prologue.hip:147`, `:156`, and the half-even rule of `:56-64`);
    * fp8 (bf16 inputs): `sk = max(RN(kmax / 448), 1e-12)`, `K8 = e4m3(min(RN(kc / sk), 448))`,
      no lower clamp (`h34_prologue.hip:158-165`);
    * `SK = sk` on live rows and `1.0` on pad rows (`h34_prologue.hip:148`).

    Returns `(K8 (BH, n_pad, D) int8 | float8_e4m3fn, SK (BH, n_pad) fp32)`.
    """
    BH, N, D = k.shape
    kf = k.to(torch.float32)
    if mean is not None:
        kf = kf - mean[:, None, :].to(torch.float32)
    kc = _pad_rows(kf, n_pad)
    kmax = kc.abs().amax(dim=2)
    if int8:
        sk = torch.maximum(kmax / I8_MAX, FLOOR)
        x = kc / sk[:, :, None]
        k8 = torch.clamp(torch.round(x), -128.0, 127.0).to(torch.int8)
    else:
        sk = torch.maximum(kmax / P_SCALE, FLOOR)
        x = torch.minimum(kc / sk[:, :, None], P_SCALE)
        k8 = x.to(F8)
    sk = sk.clone()
    sk[:, N:] = 1.0
    return k8, sk


def quant_v(v, n_pad, mean=None):
    """V per-token fp8 quantization, stored transposed (`kernels/hip/h34_prologue.hip:168-211`).

    `vmax = max_d |v|`; `sv = max(RN(vmax / 448), 1e-12)`; `SV = sv` on live rows, `0.0` on pad rows
    (`h34_prologue.hip:186`); `V8T[d, n] = e4m3(min(RN(v[n, d] / sv), 448))`, 0 on pad rows.
    With `mean` (smooth_v), `v` is first `RN(fp32(v) - mean)` on live rows, before the absmax
    (`sageattention/sk1_backend/quant_triton.py:714-719`); pad rows stay 0.

    Returns `(V8T (BH, D, n_pad) float8_e4m3fn, SV (BH, n_pad) fp32)`.
    """
    BH, N, D = v.shape
    vf = v.to(torch.float32)
    if mean is not None:
        vf = vf - mean[:, None, :].to(torch.float32)
    vf = _pad_rows(vf, n_pad)
    vmax = vf.abs().amax(dim=2)
    sv = torch.maximum(vmax / P_SCALE, FLOOR)
    x = torch.minimum(vf / sv[:, :, None], P_SCALE)
    v8t = x.to(F8).transpose(1, 2).contiguous()
    sv = sv.clone()
    sv[:, N:] = 0.0
    return v8t, sv


def fold_v_scale(sv):
    """The per-(b,h) V-scale fold (`sageattention/sk1_backend/__init__.py:561-579`).

    `S = max(max_n SV[n], 1.0)` and `SV' = RN(SV / S)`. `S == 1` exactly when every `|v| <= 448`,
    and then `SV'` is `SV` bit for bit. Returns `(S (BH,) fp32, SV' (BH, n_pad) fp32)`.
    """
    s = torch.clamp_min(sv.amax(dim=1), 1.0)
    return s, sv / s[:, None]


def quant_q(q, sm_scale, int8=True):
    """Per-query-row Q quantization done inside the reference main loop.

    int8 (`kernels/hip/sk1_t6i.hip:91-117`): `amax = max(max_d |q|, 1e-12)`; `qinv = RN(127 / amax)`;
    `Q8 = clamp(rne(RN(q * qinv)), -128, 127)` -- multiplication by a correctly rounded
    RECIPROCAL, unlike K's division; `sq = RN(amax / 127)`; `c_q = RN(RN(sm * LOG2E) * sq)`.

    fp8 (`kernels/hip/sk1_t4a1s.hip:79-105`, templated by `sk1_t4a1sb.hip`):
    `qinv = RN(448 / amax)`; `Q8 = e4m3(clamp(RN(q * qinv), -448, 448))`; `sq = RN(amax / 448)`.

    `q`: (BH, N, D) fp16/bf16. Returns `(Q8 (BH, N, D), sq (BH, N) fp32, c_q (BH, N) fp32)`.
    """
    qf = q.to(torch.float32)
    amax = torch.maximum(qf.abs().amax(dim=2), FLOOR)
    sm = torch.tensor(float(sm_scale), dtype=torch.float32)
    top = I8_MAX if int8 else P_SCALE
    qinv = top / amax
    x = qf * qinv[:, :, None]
    if int8:
        q8 = torch.clamp(torch.round(x), -128.0, 127.0).to(torch.int8)
    else:
        q8 = torch.clamp(x, -P_SCALE, P_SCALE).to(F8)
    sq = amax / top
    c_q = (sm * LOG2E) * sq
    return q8, sq, c_q


def attention_tiles(q8, c_q, k8, sk, v8t, svp, s_fold, N, causal, out_dtype, tile=BN,
                    q_chunk=2048, row0=0, lse_out=None, vmean=None):
    """The main loop's online softmax over key tiles, in the reference's phase order.

    Follows `kernels/hip/sk1_t6i.hip:162-299` (and the identical fp8 form of `sk1_t4a1s.hip`):
    per key tile of `tile` keys, in order,
    * `s = RN(fp32(sum_d Q8*K8) * RN(c_q * SK[n]))` (the int8 dot product is exact in fp32:
      |sum| <= 128^3 = 2^21 < 2^24); masked keys (causal `n > m`; non-causal `n >= N`) are -inf;
    * `m_new = max(m, max_tile s)`; `m_use = m_new`, or 0 when it is -inf; `alpha = exp2(m - m_use)`;
    * `p = exp2(s - m_use)`; `l = l*alpha + sum_tile p` (the row sum is taken before the fold);
    * `p8 = e4m3(RN(p * RN(SV'[n] * 448)))`; `acc = acc*alpha + sum_n p8 * V8[n]` in fp32;
    and the epilogue `O = T(acc * (l > 0 ? RN(S / RN(l * 448)) : 0))` (`sk1_t6i.hip:281-299`), or
    with `vmean` ((BH, D) fp32, smooth_v) `O = T(fma(acc, inv, vmean[d]))`, the kernel's
    `acc * inv + vm` (`sk1_t6i.hip:290-297`), evaluated in fp64 (where acc*inv is exact) and
    rounded to fp32.

    The GPU uses the hardware `exp2` and an unspecified MFMA accumulation order, so the output is
    pinned by tolerance, not bits. Queries are processed in chunks of `q_chunk` rows to bound
    memory; chunking queries does not change any per-row arithmetic. `row0` is the sequence index of
    the first row of `q8` (for computing a subset of rows: rows are independent).

    Shapes: q8 (BH, N, D); c_q (BH, N); k8 (BH, n_pad, D); sk, svp (BH, n_pad); v8t (BH, D, n_pad);
    s_fold (BH,). Returns O (BH, N, D) in `out_dtype`.

    `lse_out` ((BH, N) fp32, optional) receives each row's log2-domain sum `m_use + log2(l)` of
    the final tile (the quantized scores' logsumexp in exp2 units, before any smooth_k
    correction; `row_lse` turns it into the natural-log value `sageattn` returns).
    """
    BH, NQ, D = q8.shape
    n_pad = k8.shape[1]
    kf = k8.to(torch.float32)
    vf = v8t.to(torch.float32)
    sv448 = svp * P_SCALE
    out = torch.empty(BH, NQ, D, dtype=out_dtype)
    neg_inf = torch.tensor(-math.inf, dtype=torch.float32)
    for r0 in range(0, NQ, q_chunk):
        r1 = min(NQ, r0 + q_chunk)
        qf = q8[:, r0:r1].to(torch.float32)
        cq = c_q[:, r0:r1]
        rows = torch.arange(row0 + r0, row0 + r1)[:, None]
        m = torch.full((BH, r1 - r0), -math.inf, dtype=torch.float32)
        l = torch.zeros(BH, r1 - r0, dtype=torch.float32)
        acc = torch.zeros(BH, r1 - r0, D, dtype=torch.float32)
        n_tiles = n_pad // tile
        if causal:
            n_tiles = min(n_tiles, (row0 + r1 - 1) // tile + 1)
        for j in range(n_tiles):
            ks = slice(j * tile, (j + 1) * tile)
            dot = torch.matmul(qf, kf[:, ks].transpose(1, 2))
            s = dot * (cq[:, :, None] * sk[:, None, ks])
            keys = torch.arange(j * tile, (j + 1) * tile)[None, :]
            dead = (keys > rows) if causal else (keys >= N)
            s = torch.where(dead[None], neg_inf, s)
            m_new = torch.maximum(m, s.amax(dim=2))
            m_use = torch.where(m_new == -math.inf, torch.zeros_like(m_new), m_new)
            alpha = torch.exp2(m - m_use)
            p = torch.exp2(s - m_use[:, :, None])
            l = l * alpha + p.sum(dim=2)
            p8 = (p * sv448[:, None, ks]).to(F8).to(torch.float32)
            acc = acc * alpha[:, :, None] + torch.matmul(p8, vf[:, :, ks].transpose(1, 2))
            m = m_new
        inv = torch.where(l > 0, s_fold[:, None] / (l * P_SCALE), torch.zeros_like(l))
        if vmean is None:
            out[:, r0:r1] = (acc * inv[:, :, None]).to(out_dtype)
        else:
            o64 = acc.double() * inv.double()[:, :, None] + vmean.double()[:, None, :]
            out[:, r0:r1] = o64.to(torch.float32).to(out_dtype)
        if lse_out is not None:
            m_use = torch.where(m == -math.inf, torch.zeros_like(m), m)
            lse_out[:, r0:r1] = m_use + torch.log2(l)
    return out


def row_lse(lse2, q, mean, sm_scale):
    """The natural-log logsumexp `sageattn(..., return_lse=True)` returns
    (`sageattention/core.py:1437-1439` of the reference): `lse2 / 1.44269504`, plus
    `sm_scale * (q . mean)` per row when the keys were smoothed (`mean` not None; `core.py:1401-1403`
    computes the same correction as `q @ km^T`). lse2 (BH, N) fp32 from `attention_tiles`; q the
    caller's (BH, N, D) values; mean (BH, D) fp32 or None. Returns (BH, N) fp32.
    """
    lse = lse2 / torch.tensor(1.44269504, dtype=torch.float32)
    if mean is not None:
        # q . mean in fp64 (each fp16/bf16 x fp32 product is exact there), rounded once to fp32:
        # independent of how many rows one call holds, unlike an fp32 matmul's blocking
        corr = torch.matmul(q.to(torch.float64), mean.to(torch.float64)[:, :, None]).squeeze(-1)
        corr = corr.to(torch.float32)
        lse = lse + corr * torch.tensor(sm_scale, dtype=torch.float32)
    return lse


def kv_planes(B, H, H_kv, N, N_kv, is_causal):
    """For each query plane b*H + h, the K/V plane it reads: b*H_kv + h // (H // H_kv) (grouped-
    query attention, the upstream API's rule, `sageattention/core.py:824-829` of the reference,
    which also raises for H not a multiple of H_kv and for causal calls with N != N_kv)."""
    if H_kv < 1 or H % H_kv != 0:
        raise ValueError("num_qo_heads must be divisible by num_kv_heads.")
    if is_causal and N != N_kv:
        raise ValueError("causal attention requires q_len == kv_len.")
    g = H // H_kv
    return (torch.arange(B)[:, None] * H_kv + torch.arange(H)[None, :] // g).reshape(-1)


def emulate_sageattn(q, k, v, tensor_layout="HND", is_causal=False, sm_scale=None, smooth_k=True,
                     qk_int8=None, smooth_v=False, vmean_def="fp64"):
    """The whole SK1 call on the CPU, returning every intermediate.

    Routing follows `sageattention/sk1_backend/__init__.py:1161-1272`: fp16 inputs use int8 Q.K
    (`sk1_t6i`), bf16 inputs use fp8 Q.K (`sk1_t4a1sb`); `qk_int8=False` forces the fp8 form for
    fp16 inputs. `sm_scale` defaults to `D ** -0.5` (`__init__.py:1165`).

    k and v may have H_kv heads (H a multiple of H_kv) and N_kv rows (N_kv == N when causal):
    query plane b*H + h reads K/V plane `kv_planes(...)[b*H + h]`. `smooth_v` subtracts V's
    sequence mean (the same fp64-accumulated mean as K's) before quantizing V and adds it back in
    the epilogue (`quant_triton.py:668-678` of the reference; its shipped HIP prologue does not
    compute V's mean). `vmean_def="fp32_chunked"` takes V's mean as the reference's Triton path
    does instead (`vseq_mean_fp32_chunked`).

    Returns a dict with `mean, vmean, k8, sk, v8t, sv, s, svp, q8, sq, c_q, o, lse` where `o` has the
    caller's layout and dtype, `lse` is (B, H, N) fp32 (the `return_lse` output), `q8, sq, c_q`
    are per query plane (B*H, ...) and `mean, vmean, k8, sk, v8t, sv, s, svp` per K/V plane
    (B*H_kv, ...).
    """
    qq, kk, vv = (to_hnd(t, tensor_layout) for t in (q, k, v))
    B, H, N, D = qq.shape
    H_kv, N_kv = kk.shape[1], kk.shape[2]
    kvp = kv_planes(B, H, H_kv, N, N_kv, is_causal)
    BH = B * H
    if qk_int8 is None:
        qk_int8 = (q.dtype == torch.float16)
    sm = float(sm_scale if sm_scale is not None else D ** -0.5)
    n_pad = n_pad_for(N_kv)
    qr = qq.reshape(BH, N, D)
    kr, vr = (t.reshape(B * H_kv, N_kv, D) for t in (kk, vv))
    mean = kseq_mean(kr) if smooth_k else None
    k8, sk = quant_k(kr, n_pad, mean=mean, int8=qk_int8)
    if not smooth_v:
        vmean = None
    elif vmean_def == "fp32_chunked":
        vmean = vseq_mean_fp32_chunked(vr)
    else:
        vmean = kseq_mean(vr)
    v8t, sv = quant_v(vr, n_pad, mean=vmean)
    s, svp = fold_v_scale(sv)
    q8, sq, c_q = quant_q(qr, sm, int8=qk_int8)
    lse2 = torch.empty(BH, N, dtype=torch.float32)
    o = attention_tiles(q8, c_q, k8[kvp], sk[kvp], v8t[kvp], svp[kvp], s[kvp], N_kv, is_causal,
                        q.dtype, lse_out=lse2, vmean=None if vmean is None else vmean[kvp])
    o = o.view(B, H, N, D)
    if tensor_layout == "NHD":
        o = o.transpose(1, 2).contiguous()
    lse = row_lse(lse2, qr, None if mean is None else mean[kvp], sm).view(B, H, N)
    return dict(mean=mean, vmean=vmean, k8=k8, sk=sk, v8t=v8t, sv=sv, s=s, svp=svp, q8=q8, sq=sq,
                c_q=c_q, o=o,
                lse=lse, n_pad=n_pad, sm_scale=sm)


def _expand_kv_heads(x, H):
    """(B, H_kv, N_kv, D) -> (B, H, N_kv, D): query head h sees K/V head h // (H // H_kv)."""
    if x.shape[1] == H:
        return x
    if H % x.shape[1]:
        raise ValueError("num_qo_heads must be divisible by num_kv_heads.")
    return x.repeat_interleave(H // x.shape[1], dim=1)


def exact_lse(q, k, is_causal=False, sm_scale=None, tensor_layout="HND", q_chunk=1024):
    """The natural-log logsumexp of each row of Q.K^T * sm_scale, unquantized, in fp64 (the
    yardstick for `return_lse`; the reference's `_attention_lse_reference`, `core.py:424-467`).
    Returns (B, H, N) fp64."""
    qq, kk = (to_hnd(t, tensor_layout).to(torch.float64) for t in (q, k))
    B, H, N, D = qq.shape
    kk = _expand_kv_heads(kk, H)
    sm = float(sm_scale if sm_scale is not None else D ** -0.5)
    out = torch.empty(B, H, N, dtype=torch.float64)
    for r0 in range(0, N, q_chunk):
        r1 = min(N, r0 + q_chunk)
        s = torch.matmul(qq[:, :, r0:r1], kk.transpose(2, 3)) * sm
        if is_causal:
            dead = torch.arange(kk.shape[2])[None, :] > torch.arange(r0, r1)[:, None]
            s = s.masked_fill(dead, -math.inf)
        out[:, :, r0:r1] = torch.logsumexp(s, dim=-1)
    return out


def exact_attention(q, k, v, is_causal=False, sm_scale=None, tensor_layout="HND", q_chunk=1024):
    """Unquantized attention in fp64, chunked over queries (the error yardstick, not the oracle).

    Returns fp64 output in the caller's layout.
    """
    qq, kk, vv = (to_hnd(t, tensor_layout).to(torch.float64) for t in (q, k, v))
    B, H, N, D = qq.shape
    kk, vv = _expand_kv_heads(kk, H), _expand_kv_heads(vv, H)
    sm = float(sm_scale if sm_scale is not None else D ** -0.5)
    out = torch.empty(B, H, N, D, dtype=torch.float64)
    for r0 in range(0, N, q_chunk):
        r1 = min(N, r0 + q_chunk)
        s = torch.matmul(qq[:, :, r0:r1], kk.transpose(2, 3)) * sm
        if is_causal:
            dead = torch.arange(kk.shape[2])[None, :] > torch.arange(r0, r1)[:, None]
            s = s.masked_fill(dead, -math.inf)
        out[:, :, r0:r1] = torch.matmul(torch.softmax(s, dim=-1), vv)
    if tensor_layout == "NHD":
        out = out.transpose(1, 2)
    return out
