"""The per-frame arena and the kernel scratch on the MI355X.

cw_frame_alloc / cw_frame_reset are GpuContext::empty / reset_frame
(src/context.rs:207-250): every reference kernel wrapper takes its output
from this arena (e.g. q4::gemv, src/kernels/q4.rs:9-30), and the same call
sequence after a reset must get the same addresses, since the reference's
bind-group cache and this library's recorded launch sequences depend on it.
The kernel scratch of the standalone entry points may grow; a sequence
recorded before it grew must still replay correctly."""
import ctypes as C

import numpy as np
import pytest

import cw
import oracle as orc

pytestmark = pytest.mark.gpu

MB = 1 << 20


def falloc(ctx, n):
    p = C.c_void_p()
    cw.check(cw.lib().cw_frame_alloc(ctx.h, n, C.byref(p)))
    return p.value


def reset(ctx):
    cw.check(cw.lib().cw_frame_reset(ctx.h))


def test_same_sequence_same_addresses(ctx):
    """Same sizes after a reset -> same addresses; 256-byte aligned and
    disjoint; a request that no longer fits the 64 MB chunk moves to a new
    one, and the sequence stays deterministic across the growth."""
    sizes = [100, 4096, 1, 40 * MB, 40 * MB, 300, 70 * MB, 8]
    reset(ctx)
    a = [falloc(ctx, n) for n in sizes]
    reset(ctx)
    b = [falloc(ctx, n) for n in sizes]
    assert a == b
    for p in a:
        assert p % 256 == 0
    spans = sorted((p, p + n) for p, n in zip(a, sizes))
    for (lo0, hi0), (lo1, _) in zip(spans, spans[1:]):
        assert hi0 <= lo1, "overlapping frame allocations"
    # the second 40 MB does not fit after the first in a 64 MB chunk
    assert abs(a[4] - a[3]) >= 40 * MB
    reset(ctx)
    c = [falloc(ctx, n) for n in sizes]
    assert c == a


def test_growth_refused_while_recording(ctx):
    """A frame request that needs a new chunk allocates, which a recording
    may not do: CW_ERR_STATE, and the recording still closes cleanly; one
    that fits the existing chunks is served."""
    L = cw.lib()
    a = ctx.storage(np.arange(256, dtype=np.float32))
    reset(ctx)
    falloc(ctx, 1024)
    reset(ctx)
    ctx.graph_begin()
    try:
        p = C.c_void_p()
        assert L.cw_frame_alloc(ctx.h, 1024, C.byref(p)) == 0
        # one kernel into the recording, so it is not empty
        cw.check(L.cw_add(ctx.h, a.ptr, a.ptr, 256, p))
        rc = L.cw_frame_alloc(ctx.h, 512 * MB, C.byref(C.c_void_p()))
        assert rc == cw.CW_ERR_STATE
        assert "recorded" in L.cw_last_error().decode()
    finally:
        g = ctx.graph_end()
    g.launch()
    ctx.flush()
    out = np.empty(256, np.float32)
    cw.check(L.cw_download(ctx.h, out.ctypes.data_as(C.c_void_p), p, 1024))
    assert np.array_equal(out, 2 * np.arange(256, dtype=np.float32))
    g.close()
    reset(ctx)


def test_wrapper_style_gemv_through_the_arena(ctx):
    """The binding's q4::gemv wrapper: output from cw_frame_alloc, then
    cw_q4_gemv, then cw_download (GpuContext::read); after a reset the same
    wrapper call gets the same output address and the same result."""
    L = cw.lib()
    in_f, out_f = 1024, 3072
    s, q = cw.synth_q4(cw.synth_key(51, "arena.w"), out_f, in_f)
    x = cw.synth_normal_f32(cw.synth_key(51, "arena.x"), in_f)
    xd, sd, qd = ctx.storage(x), ctx.storage(s), ctx.storage(q)
    ref = orc.q4_gemv(x, s, q, in_f, out_f)

    def wrapper():
        y = falloc(ctx, out_f * 4)
        cw.check(L.cw_q4_gemv(ctx.h, xd.ptr, sd.ptr, qd.ptr, in_f, out_f, C.c_void_p(y)))
        out = np.empty(out_f, np.float32)
        cw.check(L.cw_download(ctx.h, out.ctypes.data_as(C.c_void_p), C.c_void_p(y), out_f * 4))
        return y, out

    reset(ctx)
    y0, out0 = wrapper()
    y1, out1 = wrapper()       # a second output in the same frame: another slot
    assert y1 != y0
    reset(ctx)
    y2, out2 = wrapper()
    assert y2 == y0
    for o in (out0, out1, out2):
        assert float(np.max(np.abs(o - ref)) / np.max(np.abs(ref))) <= 1e-4
    assert np.array_equal(out0, out2)


def test_recorded_sequence_survives_scratch_growth(ctx, rng):
    """Attention recorded at 300 positions uses the kernel scratch of that
    size; a later eager call at 8,000 positions makes the scratch grow (a
    fresh context, so no earlier test has grown it).  Replaying the recording
    afterwards must still give the eager result: the old scratch is kept
    alive, not freed."""
    L = cw.lib()
    nh, nkv, hd = 32, 8, 128
    big = 8000
    kh = rng.standard_normal(big * nkv * hd).astype(np.float16).view(np.uint16)
    vh = rng.standard_normal(big * nkv * hd).astype(np.float16).view(np.uint16)
    qh = (rng.standard_normal(nh * hd) * 0.3).astype(np.float32)
    with cw.Context(0) as c2:
        kc, vc, qa = c2.storage(kh), c2.storage(vh), c2.storage(qh)
        o_small, o_big = c2.empty(nh * hd), c2.empty(nh * hd)

        def small():
            cw.check(L.cw_attention(c2.h, qa.ptr, kc.ptr, vc.ptr, cw.CW_F16, nh, nkv, 300, hd,
                                    o_small.ptr))

        small()
        c2.flush()
        want = o_small.download()
        c2.graph_begin()
        small()
        g = c2.graph_end()
        cw.check(L.cw_attention(c2.h, qa.ptr, kc.ptr, vc.ptr, cw.CW_F16, nh, nkv, big, hd,
                                o_big.ptr))
        c2.flush()
        for _ in range(3):
            o_small.upload(np.zeros(nh * hd, np.float32))
            g.launch()
            c2.flush()
            assert np.array_equal(o_small.download(), want)
        g.close()
        got_big = o_big.download()
    ref = orc.attention_f64(qh, kh, vh, 1, nh, nkv, big, hd)
    assert np.max(np.abs(got_big - ref)) < 5e-5
    ref300 = orc.attention_f64(qh, kh, vh, 1, nh, nkv, 300, hd)
    assert np.max(np.abs(want - ref300)) < 5e-5
