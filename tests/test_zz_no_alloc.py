"""xe_attn_decode_dev_static (the allocation-free attention entry point)
against xe_attn_decode_dev, through the C ABI: bit-identical outputs on two
calls in a row, the second smaller, and a clear refusal of a shape whose
partials exceed the static workspace."""
import math

import numpy as np
import pytest

import oracle_lib as O

pytestmark = pytest.mark.gpu


def call(L, fn, ctx, q, k, v, lens, b, hq, hkv, hd, mc, scale, out):
    return getattr(L, fn)(ctx.h, q.ptr, k.ptr, v.ptr, lens.ptr, b, hq, hkv, hd, mc, scale, out.ptr)


def test_static_entry_matches_allocating_entry(gpu, xe):
    dev, ctx = gpu
    L = xe.lib()
    for (b, hq, hkv, hd, mc) in [(6, 4, 1, 256, 4096), (2, 12, 12, 64, 1024)]:
        print("[case] no-alloc attn b=%d hq=%d hkv=%d hd=%d ctx=%d" % (b, hq, hkv, hd, mc), flush=True)
        rng = np.random.default_rng(b * 100 + hd)
        lens = rng.integers(1, mc + 1, b).astype(np.int32)
        q = rng.standard_normal((b, hq, hd)).astype(np.float32)
        n = b * hkv * mc * hd
        kb, vb = xe.Buf(dev, n * 2), xe.Buf(dev, n * 2)
        kb.fill_synthetic(xe.XE_BF16, 77, 1, n)
        vb.fill_synthetic(xe.XE_BF16, 77, 2, n)
        qb, lb = xe.Buf.from_array(dev, q), xe.Buf.from_array(dev, lens)
        o1, o2 = xe.Buf(dev, q.nbytes), xe.Buf(dev, q.nbytes)
        scale = 1.0 / math.sqrt(hd)
        assert call(L, "xe_attn_decode_dev", ctx, qb, kb, vb, lb, b, hq, hkv, hd, mc, scale, o1) == 0, \
            xe.last_error()
        assert call(L, "xe_attn_decode_dev_static", ctx, qb, kb, vb, lb, b, hq, hkv, hd, mc, scale,
                    o2) == 0, xe.last_error()
        ctx.synchronize()
        want = o1.read(np.float32, q.size)
        got = o2.read(np.float32, q.size)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
        # and the oracle agrees on the first stream
        ks = O.bf16_bits(O.synth_range(77, 1, 0.0, 1.0, 0, hkv * mc * hd)).reshape(1, hkv, mc, hd)
        vs = O.bf16_bits(O.synth_range(77, 2, 0.0, 1.0, 0, hkv * mc * hd)).reshape(1, hkv, mc, hd)
        ref = O.attn_decode(q[:1], ks, vs, lens[:1], scale).reshape(-1)
        assert np.allclose(got[:hq * hd], ref, rtol=1e-2, atol=1e-3)
        for buf in (kb, vb, qb, lb, o1, o2):
            buf.free()


def test_static_entry_refuses_oversized_partials(gpu, xe):
    dev, ctx = gpu
    L = xe.lib()
    # 16 streams x 64 query heads x 64 splits x 258 floats > 4 Mi floats
    b, hq, hkv, hd, mc = 16, 64, 1, 256, 8192
    small = xe.Buf(dev, 4096)
    rc = L.xe_attn_decode_dev_static(ctx.h, small.ptr, small.ptr, small.ptr, small.ptr, b, hq, hkv,
                                     hd, mc, 0.0625, small.ptr)
    assert rc == -1
    assert "static" in xe.last_error() and "workspace" in xe.last_error()
    small.free()
