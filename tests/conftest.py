import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels through the C ABI)")


def gpu_available() -> bool:
    try:
        import torch
        return torch.cuda.is_available()
    except Exception:
        return False


def pytest_terminal_summary(terminalreporter, exitstatus, config):
    """The parity figures of the session: max |err| / RMS raw (nothing subtracted), net (the figure the bar applies
    to: beyond the output's own rounding against an fp32 reference, or over the elements more than one bf16 step
    from a bf16 reference) and, against bf16 references, the share of elements one step apart."""
    from tests import gen
    if not gen.RECORDS:
        return
    tr = terminalreporter
    tr.write_sep("-", "parity: max|err|/RMS(ref) raw / net (bar) / 1- and 2-step shares")
    worst_ratio = 0.0
    for tid, what, raw, net, ulp1, tol, ulp2 in gen.RECORDS:
        u = "" if ulp1 is None else f"  ulp1 {ulp1:.4f}  ulp2 {ulp2:.5f}"
        tr.write_line(f"{tid} [{what}]  raw {raw:.3e}  net {net:.3e} (<= {tol:.0e}){u}")
        worst_ratio = max(worst_ratio, net / tol)
    raws = [r[2] for r in gen.RECORDS]
    u1 = [r[4] for r in gen.RECORDS if r[4] is not None]
    tr.write_line(f"{len(gen.RECORDS)} checks; largest net/bar {worst_ratio:.3f}; largest raw {max(raws):.3e}"
                  + (f"; largest 1-ulp share {max(u1):.4f}" if u1 else ""))


@pytest.fixture(autouse=True)
def workspace_header_stays_zero(request):
    """After every GPU test: the counter header of each workspace the ops wrappers hand out is back to zero
    (ifd_workspace_check), so no split-K or fixup path left a counter behind for a later call to trip over."""
    yield
    if request.node.get_closest_marker("gpu") is None or not gpu_available():
        return
    from inferd_amd import ops
    for buf in list(ops._ws_cache.values()):
        if buf.numel() >= 4096:  # smaller buffers never carried a header
            ops.workspace_check(buf)


def pytest_collection_modifyitems(config, items):
    if gpu_available():
        return
    skip = pytest.mark.skip(reason="no GPU in this container")
    for it in items:
        if "gpu" in it.keywords:
            it.add_marker(skip)
