"""The device-layer and runtime seams of the C ABI.

* Asynchronous submission (xrt_shim.h:47-54 shim_run_*_start / wait / free):
  xe_ctx_record on queued *_dev work, xe_run_query / wait / free.
* The resident decode step (ElfResident, npu-xrt/src/lib.rs:591-629):
  open / write / dispatch (and dispatch_start) / read against the plain
  xe_decoder_step on the same weights.
* A C client (tests/c/decode_client.c, the shape of npu-capi/tests/
  c_smoke.rs): compiled with gcc against include/xdna_engine.h and linked
  against the library; without a GPU it must run host-safe, with one its
  per-stream-position and resident token streams must be the oracle's.
* The bounded-wait failure path of the low-latency step kernel, forced from
  the host (XE_LL_STALL_TEST: the end-of-step wait expects an epoch that
  never comes, XE_WAIT_LIMIT_US: a 2 ms limit): every workgroup stops at its
  own limit, the launch ends, the host reports the timeout, and the decoder
  runs correctly again afterwards.
"""
import os
import shutil
import subprocess

import numpy as np
import pytest

import oracle_lib as O
from parity_util import greedy_identity

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "xdna-engine_amd")


def build_client(tmp_path):
    if shutil.which("gcc") is None:
        pytest.skip("no gcc")
    exe = str(tmp_path / "decode_client")
    subprocess.check_call(["gcc", "-std=c99", "-Wall", "-Wextra", "-Werror", "-pedantic",
                           "-I" + os.path.join(ROOT, "include"),
                           os.path.join(ROOT, "tests", "c", "decode_client.c"),
                           "-L" + PKG, "-Wl,-rpath," + PKG, "-lxdna_engine", "-o", exe])
    return exe


def tiny_gemma(xe, max_ctx=128):
    return xe.GEMMA3_1B.replace(n_layers=2, d_model=256, ffn=1024, vocab=2048, max_ctx=max_ctx)


def oracle_cfg(cfg):
    c = O.ModelConfig()
    for name, _ in O.ModelConfig._fields_:
        setattr(c, name, getattr(cfg, name))
    return c


def test_c_client_links_and_runs_host_safe(tmp_path, xe):
    """Compiles as pedantic C99 against the header, links the library and,
    with no GPU visible, reports zero devices and exits 0."""
    exe = build_client(tmp_path)
    if xe.device_count() > 0:
        pytest.skip("a GPU is visible: the GPU test runs the client")
    out = subprocess.run([exe], capture_output=True, text=True, timeout=120)
    assert out.returncode == 0, out.stderr
    assert out.stdout.strip() == "devices=0"


@pytest.mark.gpu
def test_c_client_streams_are_the_oracles(tmp_path, xe, gpu):
    exe = build_client(tmp_path)
    n_new = 12
    print("[case] C client, 2 streams x %d tokens" % n_new, flush=True)
    # the client is a second process on the GPU this test process holds: the
    # low-latency executor's cooperative launch needs the whole device and is
    # refused there, so the client runs the graph executor
    env = dict(os.environ, XE_STEP="graph")
    out = subprocess.run([exe, str(n_new)], capture_output=True, text=True, timeout=300, env=env)
    assert out.returncode == 0, out.stderr
    lines = dict(l.split(":", 1) for l in out.stdout.strip().splitlines() if ":" in l and "=" not in l)
    prompts = np.array([[11, 503, 77, 1024, 9], [42, 42, 1999, 3, 640]], np.int32)
    for b in range(2):
        for path in ("step", "resident"):
            got = np.array([int(t) for t in lines["%s %d" % (path, b)].split()], np.int32)
            om = O.OracleModel(oracle_cfg(tiny_gemma(xe)), 7, 1)
            greedy_identity(got[None], om, prompts[b:b + 1], "c-client-%s-%d" % (path, b))
            om.close()


@pytest.mark.gpu
def test_run_handle_on_async_gemv(gpu, xe):
    """shim_run_matmul8_start = xe_gemv_dev + xe_ctx_record: the handle
    completes, and the result equals the blocking GEMV."""
    dev, ctx = gpu
    rng = np.random.default_rng(1)
    m, k, b = 4096, 4096, 4
    q = rng.integers(-127, 128, (m, k)).astype(np.int8)
    s = rng.uniform(0.001, 0.02, m).astype(np.float32)
    x = rng.standard_normal((b, k)).astype(np.float32)
    w = ctx.register_weight_q8(q, s)
    xb, yb = xe.Buf.from_array(dev, x), xe.Buf(dev, b * m * 4)
    ctx.gemv_dev(w, xb, b, yb)
    run = ctx.record()
    run.wait()
    assert run.query()
    got = yb.read(np.float32, b * m).reshape(b, m)
    run.free()
    want = ctx.gemv(w, x)
    assert np.array_equal(got, want)
    for bb in (xb, yb):
        bb.free()
    w.free()


@pytest.mark.gpu
@pytest.mark.parametrize("batch,executor", [(1, None), (3, None), (2, "graph")])
def test_resident_step_equals_decoder_step(gpu, xe, batch, executor, monkeypatch):
    """The resident step (written parameters, dispatch / dispatch_start,
    read) gives the tokens and logits of xe_decoder_step, bit for bit, on the
    low-latency executor and on the graph executor."""
    dev, _ = gpu
    if executor:
        monkeypatch.setenv("XE_STEP", executor)
    cfg = tiny_gemma(xe)
    a = xe.Decoder(dev, cfg, max_batch=batch)
    b = xe.Decoder(dev, cfg, max_batch=batch)
    a.init_synthetic(5)
    b.init_synthetic(5)
    res = xe.Resident(b, batch)
    with pytest.raises(xe.XdnaError, match="no completed dispatch"):
        res.read()
    rng = np.random.default_rng(batch)
    tok = rng.integers(0, cfg.vocab, batch).astype(np.int32)
    pos = np.arange(batch, dtype=np.int32)  # per-stream positions
    for i in range(10):
        la, na = a.step(tok, pos)
        res.write(tok, pos)
        if i % 2:
            res.dispatch()
        else:
            run = res.dispatch_start()
            with pytest.raises(xe.XdnaError, match="in flight"):
                res.write(tok, pos)
            run.wait()
            run.free()
        nb, lb = res.read(want_logits=True)
        assert np.array_equal(na, nb), i
        assert np.array_equal(la.view(np.uint32), lb.view(np.uint32)), i
        tok, pos = na, pos + 1
    res.close()
    a.close()
    b.close()


@pytest.mark.gpu
def test_ll_bounded_wait_failure_is_reported_and_recoverable(gpu, xe, monkeypatch):
    """Forced from the host: the low-latency kernel's end-of-step wait never
    sees its epoch; each workgroup gives up at its 2 ms limit, sets the
    status word, the launch ends, and the step reports the timeout.  With
    the hook off the decoder then decodes the oracle's stream again."""
    dev, _ = gpu
    cfg = tiny_gemma(xe)
    dec = xe.Decoder(dev, cfg, max_batch=1)
    dec.init_synthetic(7)
    assert dec.executor(1) == "ll"
    monkeypatch.setenv("XE_LL_STALL_TEST", "1")
    monkeypatch.setenv("XE_WAIT_LIMIT_US", "2000")
    print("[case] LL stalled wait, 2 ms limit", flush=True)
    with pytest.raises(xe.XdnaError, match="low-latency step kernel: an exchange wait timed out"):
        dec.step(np.array([3], np.int32), np.array([0], np.int32))
    monkeypatch.delenv("XE_LL_STALL_TEST")
    monkeypatch.delenv("XE_WAIT_LIMIT_US")
    dec.reset()
    prompt = np.array([[11, 503, 77, 1024]], np.int32)
    got = dec.generate(prompt, 8)
    om = O.OracleModel(oracle_cfg(cfg), 7, 1)
    greedy_identity(got, om, prompt, "ll-after-timeout")
    om.close()
    dec.close()
