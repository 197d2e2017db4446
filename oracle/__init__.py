"""CPU oracle for the SageAttention SK1 quantized-attention path.

TEST INFRASTRUCTURE ONLY. Nothing in the product imports this package. Only `tests/`,
`__graft_entry__.smoke()` and the `cpu_baseline` leg of `bench.py` may import it, and only as the
checker (or, for `cpu_baseline`, as the CPU restatement that is timed). The product path
(`sageattention.sageattn`) runs the gfx950 HIP library and raises when it is missing.

`sage_scheme` restates the reference scheme in PyTorch-CPU fp32 with one operation per rounding.
Every function cites the reference file and lines it follows (paths relative to the reference
repository root).
"""
from .sage_scheme import (  # noqa: F401
    BN, FLOOR, LOG2E, P_SCALE, I8_MAX,
    n_pad_for, kseq_mean, quant_k, quant_v, fold_v_scale, quant_q, attention_tiles,
    emulate_sageattn, exact_attention, exact_lse, kv_planes, row_lse, to_hnd,
    vseq_mean_fp32_chunked,
)
