import os
import subprocess
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
GOLDEN = os.path.join(ROOT, "tests", "golden")
sys.path.insert(0, ROOT)
sys.path.insert(0, GOLDEN)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) device")


@pytest.fixture(scope="session")
def oracle():
    from oracle import bind
    if not os.path.exists(bind.ORACLE_PATH):  # build only when nothing is built
        subprocess.run(["make", "-s", "-C", os.path.join(ROOT, "oracle"), bind.ORACLE_PATH], check=True)
    return bind.Oracle()


@pytest.fixture(scope="session")
def ref():
    from oracle import bind
    if not bind.ref_available():
        pytest.skip("oracle/_ref (the compiled reference) is not built here")
    r = bind.Ref()
    if not r.cpu_ok():
        pytest.skip("this CPU lacks the reference's AVX-512 VNNI/BF16")
    r.set_threads(min(8, os.cpu_count() or 1))
    return r


@pytest.fixture(scope="session")
def golden():
    def load(name):
        return np.load(os.path.join(GOLDEN, name), allow_pickle=False)
    return load


@pytest.fixture(scope="session")
def synth_lib():
    from malkin_amd import synth
    if not os.path.exists(synth.LIB_PATH):
        from malkin_amd import build
        build.build_synth()
    return synth


@pytest.fixture(scope="session")
def model_files(tmp_path_factory, synth_lib):
    """The golden models' GGUF files, regenerated from their recorded configs (tests/golden/make_golden.py)."""
    import make_golden
    d = str(tmp_path_factory.mktemp("models"))
    return {name: make_golden.model_path(d, name) for name in make_golden.MODEL_CFGS}


@pytest.fixture(scope="session")
def mk():
    """A device context. Raises (no silent fallback) when the native library is missing."""
    import malkin_amd
    malkin_amd.load()
    try:
        ctx = malkin_amd.Context(0)
    except malkin_amd.MkError as e:
        if e.code == malkin_amd.MK_ERR_NO_DEVICE:
            pytest.skip("no HIP device")
        raise
    yield ctx
    ctx.close()
