import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for path in (ROOT, os.path.join(ROOT, "algebraic-extra_amd")):
    if path not in sys.path:
        sys.path.insert(0, path)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a real MI355X (gfx950) and the built HIP library")


def pytest_collection_modifyitems(config, items):
    # GPU tests run only when a GPU is present; on CPU boxes `-m "not gpu"`
    # deselects them, and without a GPU an explicit `-m gpu` run skips them.
    try:
        import torch
        has_gpu = torch.cuda.is_available()
    except Exception:  # pragma: no cover
        has_gpu = False
    if has_gpu:
        return
    import pytest
    skip = pytest.mark.skip(reason="no GPU in this container")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


def pytest_terminal_summary(terminalreporter):
    """The bf16 comparisons of the session against the fixed 2e-2 max-abs
    bound (the tests allow one bf16 ulp of max|b| once that exceeds 2e-2)."""
    _tol = sys.modules.get("_tol")  # the module the tests import (tests/ is on sys.path)
    if _tol is None:
        return
    recs = _tol.BF16_RECORDS
    if not recs:
        return
    within = sum(1 for _, mae, _, _ in recs if mae <= _tol.BF16_MAX_ABS)
    tr = terminalreporter
    tr.write_sep("-", "bf16 parity: max-abs against 2e-2")
    tr.write_line(f"{len(recs)} bf16 comparisons; {within} within max-abs {_tol.BF16_MAX_ABS}; "
                  f"worst rel-L2 {max(r for *_, r in recs):.3e}")
    worst = sorted(recs, key=lambda x: -x[1])[:8]
    for what, mae, mb, r in worst:
        ulp = _tol.bf16_ulp(mb)
        tr.write_line(f"  {what or '?'}: max-abs {mae:.3e} = {mae / ulp if ulp else 0:.2f} ulp of "
                      f"max|b| {mb:.3e}, rel-L2 {r:.3e}")
