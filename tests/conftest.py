"""Shared pytest setup: import paths, the `gpu` marker and seeded input builders."""
import os
import sys

import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "ds-flashdmla-moe_amd")
for p in (ROOT, PKG):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) device and the built HIP library")


@pytest.fixture
def gpu():
    """Skips only when no GPU is present; a missing library on a GPU box is a failure."""
    if not torch.cuda.is_available():
        pytest.skip("no GPU in this environment")
    return torch.device("cuda:0")


def seeded(shape, seed, scale=1.0, dtype=torch.float32):
    """N(0, 1) * scale from torch.Generator().manual_seed(seed), generated on the CPU."""
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g, dtype=torch.float32) * scale).to(dtype)


# Tolerances of the north-star parity bar: bf16 outputs within 2e-2 max-abs and 1e-2 mean-rel
# (mean|out - ref| / mean|ref|) of the fp32 oracle; statistics m within 1e-3 max-abs and l
# within 1e-3 max-rel.
OUT_MAX_ABS = 2e-2
OUT_MEAN_REL = 1e-2
STAT_TOL = 1e-3


def assert_out_close(out, ref, what="output"):
    out = out.float()
    ref = ref.float().to(out.device)
    assert torch.isfinite(out).all(), f"{what}: non-finite values"
    diff = (out - ref).abs()
    max_abs = diff.max().item()
    mean_rel = (diff.mean() / ref.abs().mean().clamp_min(1e-30)).item()
    assert max_abs <= OUT_MAX_ABS, f"{what}: max-abs {max_abs:.3e} > {OUT_MAX_ABS}"
    assert mean_rel <= OUT_MEAN_REL, f"{what}: mean-rel {mean_rel:.3e} > {OUT_MEAN_REL}"
    return max_abs, mean_rel


def assert_stats_close(m, l, m_ref, l_ref):
    m_ref = m_ref.float().to(m.device)
    l_ref = l_ref.float().to(l.device)
    finite = torch.isfinite(m_ref)
    assert torch.equal(torch.isfinite(m), finite), "m: -inf pattern differs"
    dm = (m[finite] - m_ref[finite]).abs().max().item() if finite.any() else 0.0
    pos = l_ref > 0
    dl = ((l[pos] - l_ref[pos]).abs() / l_ref[pos]).max().item() if pos.any() else 0.0
    assert torch.all(l[~pos] == 0), "l: rows without keys must be 0"
    assert dm <= STAT_TOL, f"m: max-abs {dm:.3e} > {STAT_TOL}"
    assert dl <= STAT_TOL, f"l: max-rel {dl:.3e} > {STAT_TOL}"
    return dm, dl
