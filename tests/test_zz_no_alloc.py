"""cw_attention_noalloc (no counterpart in the reference; for callers that
cannot allocate) against cw_attention, through the C ABI: two calls in a
row, the second with a smaller input, each bit-identical to the allocating
entry point's result on the same inputs (one kernel, one reduction order)
and within the attention bar of the oracle; a size beyond the static scratch
is refused with an error."""
import ctypes as C

import numpy as np
import pytest

import cw
import oracle as orc

pytestmark = pytest.mark.gpu


def run(ctx, fn, q, kc, vc, kv_dtype, nh, nkv, seq, hd):
    out = ctx.empty(nh * hd)
    cw.check(fn(ctx.h, q.ptr, kc.ptr, vc.ptr, kv_dtype, nh, nkv, seq, hd, out.ptr))
    ctx.flush()
    return out.download()


@pytest.mark.parametrize("kv_dtype", [cw.CW_F16, cw.CW_F32])
def test_noalloc_matches_allocating_entry(ctx, kv_dtype):
    L = cw.lib()
    rng = np.random.default_rng(77 + kv_dtype)
    nh, nkv, hd = 32, 8, 128
    for seq in (4352, 1000):  # the second call smaller than the first
        print(f"\n[noalloc] kv_dtype={kv_dtype} seq={seq}", flush=True)
        kh = rng.standard_normal(seq * nkv * hd).astype(np.float32)
        vh = rng.standard_normal(seq * nkv * hd).astype(np.float32)
        if kv_dtype == cw.CW_F16:
            kh = kh.astype(np.float16).view(np.uint16)
            vh = vh.astype(np.float16).view(np.uint16)
        qh = (rng.standard_normal(nh * hd) * 0.3).astype(np.float32)
        kc, vc, q = ctx.storage(kh), ctx.storage(vh), ctx.storage(qh)
        want = run(ctx, L.cw_attention, q, kc, vc, kv_dtype, nh, nkv, seq, hd)
        got = run(ctx, L.cw_attention_noalloc, q, kc, vc, kv_dtype, nh, nkv, seq, hd)
        assert np.array_equal(got, want), float(np.max(np.abs(got - want)))
        ref = orc.attention_f64(qh, kh, vh, int(kv_dtype == cw.CW_F16), nh, nkv, seq, hd)
        assert np.max(np.abs(got - ref)) < 5e-5
        for d in (kc, vc, q):
            ctx.free(d)


def test_noalloc_refuses_beyond_its_scratch(ctx):
    L = cw.lib()
    nh, nkv, hd, seq = 32, 8, 128, 8200  # 32 * 513 * 130 * 4 bytes > 8 MiB
    buf = ctx.empty(16)
    rc = L.cw_attention_noalloc(ctx.h, buf.ptr, buf.ptr, buf.ptr, cw.CW_F16, nh, nkv, seq, hd,
                                buf.ptr)
    assert rc == cw.CW_ERR_ARG
    assert "static scratch" in L.cw_last_error().decode()


def test_noalloc_first_call_recorded_on_a_fresh_context():
    """The first attention call of a fresh context is cw_attention_noalloc
    inside a recording: it must not need the context scratch (whose growth
    is refused while recording).  Every replay of the recording, with eager
    allocating calls and synchronisations between the replays, gives the
    eager cw_attention result bit for bit."""
    L = cw.lib()
    rng = np.random.default_rng(4242)
    nh, nkv, hd, seq = 32, 8, 128, 3000
    kh = rng.standard_normal(seq * nkv * hd).astype(np.float16).view(np.uint16)
    vh = rng.standard_normal(seq * nkv * hd).astype(np.float16).view(np.uint16)
    qh = (rng.standard_normal(nh * hd) * 0.3).astype(np.float32)
    sentinel = np.full(nh * hd, np.nan, np.float32)
    with cw.Context(0) as fresh:
        kc, vc, q = fresh.storage(kh), fresh.storage(vh), fresh.storage(qh)
        out_rec = fresh.storage(sentinel)
        print(f"\n[noalloc] recorded first call, seq={seq}", flush=True)
        fresh.graph_begin()
        cw.check(L.cw_attention_noalloc(fresh.h, q.ptr, kc.ptr, vc.ptr, cw.CW_F16, nh, nkv, seq,
                                        hd, out_rec.ptr))
        g = fresh.graph_end()
        try:
            want = None
            for rep in range(3):
                out_rec.upload(sentinel)
                g.launch()
                fresh.flush()
                got = out_rec.download()
                # eager allocating call between replays (grows the context scratch)
                eager = run(fresh, L.cw_attention, q, kc, vc, cw.CW_F16, nh, nkv, seq, hd)
                if want is None:
                    want = eager
                    ref = orc.attention_f64(qh, kh, vh, 1, nh, nkv, seq, hd)
                    assert np.max(np.abs(want - ref)) < 5e-5
                assert np.array_equal(eager, want)
                assert np.array_equal(got, want), (rep, float(np.nanmax(np.abs(got - want))))
        finally:
            g.close()
