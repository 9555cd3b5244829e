"""Operator pairs for trial-driver fixtures and tests.

Every model here computes with operations that round identically on the
CPU and on the GPU: fp32 elementwise add and multiply, each rounded on its
own; conversions; slicing. Parameters and inputs come from the CPU generator.
So the reference's trial on the CPU and the device trial produce bit-identical
outputs, and their verdicts must match exactly.
"""

from __future__ import annotations

import torch


def generate_inputs(shape):
    n = int(shape["n"])
    x = torch.randn(n)
    y = torch.randn(n)
    return x, y


class _Base(torch.nn.Module):
    def __init__(self, shape):
        super().__init__()
        self.w = torch.nn.Parameter(torch.randn(int(shape["n"])))


class ScaleAdd(_Base):
    """x * w + y in fp32."""

    def forward(self, x, y):
        return x * self.w + y


class ScaleAddPerturbed(_Base):
    """ScaleAdd with every 97th element pushed by 1e-2 (fails fp32 tolerances there)."""

    def forward(self, x, y):
        out = x * self.w + y
        bump = torch.zeros_like(out)
        bump[::97] = 1e-2
        return out + bump


class ScaleAddBf16(_Base):
    """ScaleAdd rounded to bf16."""

    def forward(self, x, y):
        return (x * self.w + y).to(torch.bfloat16)


class ScaleAddBf16Coarse(_Base):
    """ScaleAdd in bf16 with the product computed from bf16 operands (a few ULP off the reference)."""

    def forward(self, x, y):
        return (x.to(torch.bfloat16) * self.w.to(torch.bfloat16) + y.to(torch.bfloat16))


class PairOut(_Base):
    """A tuple: (fp32 sum, int32 truncation of 10 * x)."""

    def forward(self, x, y):
        return x * self.w + y, (x * 10.0).to(torch.int32)


class PairOutIntOff(_Base):
    """PairOut whose integer output is off by 2 at every 50th element."""

    def forward(self, x, y):
        q = (x * 10.0).to(torch.int32)
        q[::50] += 2
        return x * self.w + y, q


class Truncated(_Base):
    """ScaleAdd without its last element (a shape mismatch)."""

    def forward(self, x, y):
        return (x * self.w + y)[:-1]


class ListOut(_Base):
    """A list of three outputs plus a non-tensor leaf."""

    def forward(self, x, y):
        return [x + y, x * self.w, (y * 2.0).to(torch.float16), 7]


class ListOutNan(_Base):
    """ListOut with NaN at every 1000th element of its second output."""

    def forward(self, x, y):
        b = x * self.w
        b[::1000] = float("nan")
        return [x + y, b, (y * 2.0).to(torch.float16), 7]


MODELS = {cls.__name__: cls for cls in (ScaleAdd, ScaleAddPerturbed, ScaleAddBf16, ScaleAddBf16Coarse, PairOut,
                                        PairOutIntOff, Truncated, ListOut, ListOutNan)}

# (name, generated model, reference model, n, policy spec or None, tolerance policy or None)
TRIAL_CASES = [
    ("identical_fp32", "ScaleAdd", "ScaleAdd", 50_000, None, None),
    ("perturbed_fp32", "ScaleAddPerturbed", "ScaleAdd", 50_000, None, None),
    ("perturbed_fp32_cosine", "ScaleAddPerturbed", "ScaleAdd", 50_000,
     {"category": "gemm", "op_name": "matmul", "config": {}}, None),
    ("bf16_coarse_default", "ScaleAddBf16Coarse", "ScaleAddBf16", 65_536, None, None),
    ("bf16_coarse_tolerant", "ScaleAddBf16Coarse", "ScaleAddBf16", 65_536,
     {"category": "activation", "op_name": "gelu", "config": {"policy": "tolerant"}},
     {"BF16": {"rtol": 1e-3, "atol": 1e-3}}),
    ("tuple_identical", "PairOut", "PairOut", 20_000, None, None),
    ("tuple_int_off", "PairOutIntOff", "PairOut", 20_000, None, None),
    ("shape_mismatch", "Truncated", "ScaleAdd", 4_096, None, None),
    ("list_identical", "ListOut", "ListOut", 30_000, None, None),
    ("list_nan", "ListOutNan", "ListOut", 30_000, None, None),
    ("large_sampled", "ScaleAddPerturbed", "ScaleAdd", 1_500_000, None, None),
]

INPUT_SEED = 1024 + 3 * 1000 + 1   # the reference's seeds for case 3, trial 1 (GCR:1362-1363)
PARAM_SEED = INPUT_SEED + 10_000_000
