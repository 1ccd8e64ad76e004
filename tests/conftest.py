import importlib.util
import pathlib
import sys

import pytest

ROOT = pathlib.Path(__file__).resolve().parent.parent
PKG_NAME = "r9700_lru_expert_cache_amd"
PKG_DIR = ROOT / "r9700-lru-expert-cache_amd"
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def load_pkg():
    """Import the package directory (its name is not a Python identifier) as PKG_NAME."""
    if PKG_NAME in sys.modules:
        return sys.modules[PKG_NAME]
    spec = importlib.util.spec_from_file_location(
        PKG_NAME, PKG_DIR / "__init__.py", submodule_search_locations=[str(PKG_DIR)])
    mod = importlib.util.module_from_spec(spec)
    sys.modules[PKG_NAME] = mod
    spec.loader.exec_module(mod)
    return mod


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a real MI355X (HIP device)")


@pytest.fixture(scope="session")
def pkg():
    return load_pkg()


def gpu_case(msg: str) -> None:
    """Name the case before each GPU step, flushed, so a fault still says what ran."""
    print(f"[gpu-case] {msg}", flush=True)


def check_argmax(got, ref, what: str, max_ties: int = 1) -> int:
    """Per-row argmax of a kernel's logits against the reference's. A row may pick another
    index only when that index is in the reference's top two and the two reference logits lie
    within one bf16 step (2^-7 relative) of each other; each such row is printed, and at most
    max_ties rows of one call may take that branch. Returns the number of such rows."""
    import numpy as np
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    am, ar = got.argmax(1), ref.argmax(1)
    ties = []
    for r in np.nonzero(am != ar)[0]:
        top2 = np.argpartition(ref[r], -2)[-2:]
        assert am[r] in top2, f"{what}: row {r} argmax {am[r]} not in the reference top two {top2}"
        gap = ref[r, ar[r]] - ref[r, am[r]]
        assert gap <= 2 ** -7 * abs(ref[r, ar[r]]), f"{what}: row {r} gap {gap:.3e}"
        ties.append((int(r), int(am[r]), int(ar[r]), float(gap)))
    if ties:
        print(f"[argmax] {what}: near-tie rows (row, got, ref, gap) {ties}", flush=True)
    assert len(ties) <= max_ties, f"{what}: {len(ties)} near-tie rows > {max_ties}"
    return len(ties)
