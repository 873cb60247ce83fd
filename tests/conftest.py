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


# ---- parity record summary (tests/parity_util.py appends one JSON line per
# comparison): printed at the end of every run, -q included, so near-ties,
# streams parted at ties and the worst logit differences show in the log ----
_PARITY_START = {}


def pytest_sessionstart(session):
    from parity_util import parity_log_path
    path = parity_log_path()
    _PARITY_START["path"] = path
    _PARITY_START["offset"] = os.path.getsize(path) if os.path.exists(path) else 0


def pytest_terminal_summary(terminalreporter, exitstatus, config):
    import json
    path = _PARITY_START.get("path")
    if not path or not os.path.exists(path):
        return
    with open(path) as f:
        f.seek(_PARITY_START.get("offset", 0))
        recs = [json.loads(line) for line in f if line.strip()]
    if not recs:
        return
    streams = [r for r in recs if "streams" in r and "tokens" in r]
    parted = sum(len(r.get("parted_at_ties", [])) for r in streams)
    diverged = sum(1 for r in recs if "diverged_stream" in r)
    forced_ties = sum(r.get("near_ties", 0) for r in recs)
    mism = sum(1 for r in recs if "argmax_mismatch_stream" in r)
    replay = [r for r in recs if "replay_tokens" in r]
    logit = [r for r in recs if "logits_rel_l2" in r]
    tw = terminalreporter
    tw.write_sep("-", "parity record (%s)" % path)
    if streams:
        mm = min(r["min_margin"] for r in streams)
        tw.write_line("greedy comparisons %d (%d stream-tokens): %d streams parted at near-ties, "
                      "%d diverged beyond them; smallest oracle top-2 margin %.3g"
                      % (len(streams), sum(r["streams"] * r["tokens"] for r in streams), parted,
                         diverged, mm))
    if replay:
        tot = sum(r["replay_tokens"] for r in replay)
        ex = sum(r["exact"] for r in replay)
        tw.write_line("oracle replays: %d tokens, %d the oracle's argmax, worst deficit %.3g"
                      % (tot, ex, max(r["worst_deficit"] for r in replay)))
    tw.write_line("teacher-forced near-ties (argmax within 2x the logit difference): %d; "
                  "argmax mismatches beyond: %d" % (forced_ties, mism))
    if logit:
        worst = max(logit, key=lambda r: r["logits_rel_l2"])
        worst_abs = max(logit, key=lambda r: r["max_abs"])
        tw.write_line("logit comparisons %d: worst rel-L2 %.3g (%s), worst max |d| %.3g (%s)"
                      % (len(logit), worst["logits_rel_l2"], worst["label"], worst_abs["max_abs"],
                         worst_abs["label"]))
