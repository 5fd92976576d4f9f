"""Recorded launch sequences (cw_graph_*, the counterpart of the reference's
per-frame replay, context.rs:141-151,330-334): a recorded sequence of kernel
calls replayed several times, with eager uploads and synchronisation between
the replays, gives exactly what the same calls give eagerly; calls that would
allocate or synchronise, the model's among them, are refused while recording."""
import numpy as np
import pytest

import cw

pytestmark = pytest.mark.gpu


def test_recorded_sequence_replays_like_eager(ctx, rng):
    L = cw.lib()
    K, N = 1024, 3072
    nh, nkv, hd, seq = 32, 8, 128, 300
    s, q = cw.synth_q4(cw.synth_key(91, "g.w"), N, K)
    sd, qd = ctx.storage(s), ctx.storage(q)
    w = ctx.storage(rng.standard_normal(K).astype(np.float32))
    r = ctx.storage(rng.standard_normal(N).astype(np.float32))
    kc = ctx.storage(rng.standard_normal(seq * nkv * hd).astype(np.float16).view(np.uint16))
    vc = ctx.storage(rng.standard_normal(seq * nkv * hd).astype(np.float16).view(np.uint16))
    x = ctx.empty(K)
    qa = ctx.empty(nh * hd)
    a, b, c = ctx.empty(K), ctx.empty(N), ctx.empty(N)
    idx = ctx.empty(1, np.uint32)
    o = ctx.empty(nh * hd)

    def sequence():
        cw.check(L.cw_rmsnorm(ctx.h, x.ptr, w.ptr, 1, K, 1e-6, a.ptr))
        cw.check(L.cw_q4_gemv(ctx.h, a.ptr, sd.ptr, qd.ptr, K, N, b.ptr))
        cw.check(L.cw_add(ctx.h, b.ptr, r.ptr, N, c.ptr))
        cw.check(L.cw_argmax(ctx.h, c.ptr, N, idx.ptr))
        cw.check(L.cw_attention(ctx.h, qa.ptr, kc.ptr, vc.ptr, cw.CW_F16, nh, nkv, seq, hd,
                                o.ptr))

    def inputs(i):
        x.upload(rng.standard_normal(K).astype(np.float32) * (1 + i))
        qa.upload(rng.standard_normal(nh * hd).astype(np.float32) * 0.3)

    def results():
        ctx.flush()
        return c.download(), idx.download(), o.download()

    inputs(0)
    sequence()  # first use: scratch and counters at these sizes
    results()
    ctx.graph_begin()
    with pytest.raises(cw.CwError, match="while a graph is being recorded"):
        ctx.flush()
    sequence()
    g = ctx.graph_end()
    for i in range(4):
        inputs(i + 1)
        sequence()
        want = results()
        g.launch()
        got = results()
        for gv, wv in zip(got, want):
            assert np.array_equal(gv.view(np.uint32), wv.view(np.uint32)), i
    g.close()
    with pytest.raises(cw.CwError, match="no recording is open"):
        ctx.graph_end()


def test_recording_refuses_a_first_allocation(ctx, rng):
    """A kernel whose scratch would have to grow cannot be recorded: the
    error names the cause and the recording can still be closed."""
    L = cw.lib()
    nh, nkv, hd, seq = 64, 64, 256, 32768  # 135 MB of partials: more than any earlier call
    qa = ctx.empty(nh * hd)
    kc = ctx.empty(16, np.uint16)  # never read: the call stops before its launch
    o = ctx.empty(nh * hd)
    ctx.graph_begin()
    with pytest.raises(cw.CwError, match="scratch must grow"):
        cw.check(L.cw_attention(ctx.h, qa.ptr, kc.ptr, kc.ptr, cw.CW_F16, nh, nkv, seq, hd,
                                o.ptr))
    g = ctx.graph_end()
    g.close()


def test_recording_refuses_model_calls(ctx):
    """Model calls synchronise or allocate: each is refused while a recording
    is open, leaves the model as it was, and works again once it is closed."""
    cfg = cw.make_config(2, 256, 4, 2, 128, 512, 64, 16, cw.CW_F16, 1e-6, 1e6)
    m = cw.Model(ctx, cfg)
    m.load_synthetic(7)
    m.finalize()
    want = m.step(3, 0)
    ctx.graph_begin()
    for call in (lambda: m.step(3, 0), lambda: m.set_taps(True),
                 lambda: m.decode_async(1, mode=cw.STEP_GRAPH), lambda: m.prefill([1, 2]),
                 lambda: cw.Model(ctx, cfg)):
        with pytest.raises(cw.CwError, match="while a graph is being recorded"):
            call()
    ctx.graph_end().close()
    assert m.step(3, 0) == want
    m.close()
