"""pytest configuration: the `gpu` marker and session fixtures.

`-m "not gpu"` runs everything that needs no GPU (oracle pinning, host logic,
the C-ABI contract and symbol checks). `-m gpu` runs the parity tests proper;
they call the engine through its C-ABI and fail (not skip) if no GPU is
visible, so a GPU run can never pass on a silent fallback.
"""

from __future__ import annotations

import pytest

import helpers


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU; parity tests proper")


@pytest.fixture(scope="session")
def pkg():
    helpers.ensure_built()
    return helpers.load_package()


@pytest.fixture(scope="session")
def eng(pkg):
    return pkg.Engine()


@pytest.fixture(scope="session")
def orc():
    helpers.ensure_built()
    return helpers.oracle(0)


@pytest.fixture(scope="session")
def gpu(eng):
    n = eng.device_count()
    assert n > 0, "no GPU visible to the engine: GPU tests must run on the MI355X box"
    arch = eng.device_arch()
    assert arch.startswith("gfx950"), f"engine is built for gfx950, device reports {arch}"
    return eng
