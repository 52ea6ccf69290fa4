"""The 16-bit parity rule (test_gpu_parity.close) on planted outputs (CPU).

The allowance beyond the tolerance exists only where half an ulp of the output
type exceeds it (fp16 |x| >= 4, bf16 |x| >= 8) and is at most that half ulp.
"""
import pytest
import torch

from test_gpu_parity import close


@pytest.mark.parametrize("dtype,ref,out,ok", [
    # outputs are exactly representable in their dtype
    # bf16: tolerance 2e-2; half ulp 1.56e-2 in [4,8), 3.1e-2 in [8,16)
    (torch.bfloat16, 5.012, 5.03125, True),
    (torch.bfloat16, 5.0, 5.03125, False),            # one ulp off below 8: no allowance
    (torch.bfloat16, 7.99, 8.0625, False),            # rounded across the edge, then one more ulp
    (torch.bfloat16, 9.0, 9.0625, False),             # one ulp in [8,16) > 2e-2 + half ulp
    (torch.bfloat16, 9.02, 9.0625, True),             # 4.25e-2 <= 5.1e-2
    (torch.bfloat16, -12.01, -12.0625, False),        # 5.25e-2 > 5.1e-2
    (torch.bfloat16, -12.02, -12.0625, True),
    # fp16: tolerance 1e-3; half ulp 0.98e-3 in [2,4), 1.95e-3 in [4,8)
    (torch.float16, 3.0, 3.001953125, False),         # one ulp in [2,4): no allowance
    (torch.float16, 3.0011, 3.001953125, True),
    (torch.float16, 5.0, 5.00390625, False),          # one ulp in [4,8) > 1e-3 + half ulp
    (torch.float16, 5.001, 5.00390625, True),         # 2.91e-3 <= 2.95e-3
    (torch.float32, 1.0, 1.0 + 2e-5, False),
    (torch.float32, 1.0, float("nan"), False),       # NaN never passes
    (torch.bfloat16, 9.0, float("nan"), False),
    (torch.float32, 1.0, 1.0 + 5e-6, True),
])
def test_rule(dtype, ref, out, ok):
    g = torch.tensor([out], dtype=torch.float32).to(dtype)
    if dtype != torch.float32 and out == out:
        assert g.float().item() == out
    r = torch.tensor([ref], dtype=torch.float32)
    if ok:
        close(g, r, dtype, "planted")
    else:
        with pytest.raises(AssertionError):
            close(g, r, dtype, "planted")
