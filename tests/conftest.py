"""pytest configuration: the `gpu` marker, and loaders for the product mirror
(xdna-engine_amd/xdna_engine.py over libxdna_engine.so) and the CPU oracle."""
import importlib.util
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
TESTS = os.path.dirname(os.path.abspath(__file__))
if TESTS not in sys.path:
    sys.path.insert(0, TESTS)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs on the GPU box)")


def load_xe():
    """Import the host mirror from the hyphenated package directory."""
    name = "xdna_engine"
    if name in sys.modules:
        return sys.modules[name]
    path = os.path.join(ROOT, "xdna-engine_amd", "xdna_engine.py")
    spec = importlib.util.spec_from_file_location(name, path)
    mod = importlib.util.module_from_spec(spec)
    sys.modules[name] = mod
    spec.loader.exec_module(mod)
    return mod


@pytest.fixture(scope="session")
def xe():
    return load_xe()


@pytest.fixture(scope="session")
def oracle():
    import oracle_lib
    oracle_lib.lib()
    return oracle_lib


@pytest.fixture(scope="session")
def gpu(xe):
    """(Device, CtxDecode) on cuda:0.  Only `gpu`-marked tests use it."""
    n = xe.device_count()
    if n <= 0:
        pytest.fail("no GPU visible to libxdna_engine.so: %s" % xe.last_error())
    dev = xe.Device(0)
    ctx = xe.CtxDecode(dev)
    print("[gpu] device", dev.name(), flush=True)
    yield dev, ctx
    ctx.close()
    dev.close()
