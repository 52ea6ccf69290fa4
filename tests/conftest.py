import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP device); run with -m gpu")


@pytest.fixture(scope="session")
def gpu():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    return torch.device("cuda", 0)


def pytest_terminal_summary(terminalreporter):
    """Per test, how many 16-bit elements took the half-ulp allowance of the
    parity rule (test_gpu_parity.close) out of those checked."""
    mod = sys.modules.get("test_gpu_parity")
    rec = getattr(mod, "FORGIVEN", None) if mod else None
    rec = {k: v for k, v in (rec or {}).items() if "test_parity_rule" not in k}  # planted cases
    if not rec:
        return
    checked = sum(v[0] for v in rec.values())
    forgiven = sum(v[1] for v in rec.values())
    terminalreporter.section("16-bit parity: elements under the half-ulp allowance")
    terminalreporter.write_line(f"total: {forgiven} of {checked} elements checked, in "
                                f"{sum(1 for v in rec.values() if v[1])} of {len(rec)} tests")
    for k, (n, f) in sorted(rec.items()):
        if f:
            terminalreporter.write_line(f"  {k}: {f} of {n}")
