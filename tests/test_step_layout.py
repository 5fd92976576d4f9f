"""CPU check of the fused decode step's buffer layout (cw_step_layout_check).

The check lays out every buffer cw_model_create and the fused step allocate,
at addresses that are never mapped, then walks the step kernel's own phase
table and requires every range a phase reads or writes to lie inside one
allocation.  With gate and up as two allocations (split_gate_up) while the
step reads them as one [2*hidden][dim] matrix, the gate|up phase of layer 0
runs `hidden` rows past the gate matrix: the check must name that range.
The model's own layout (gate|up in one allocation) must pass for every
shape the GPU tests run the fused step on.  The check also covers the
device argument block and layer table the kernel reads, the dynamic and
static LDS every phase touches, the per-workgroup argmax slots of a grid of
one workgroup per CU, the grid counters and, when tracing, the stamps."""
import pytest

import cw

N_CU = 256


def small128(max_seq, kv_dtype=cw.CW_F32, n_heads=4, n_kv=2):
    return cw.make_config(2, 256, n_heads, n_kv, 128, 512, 1000, max_seq, kv_dtype, 1e-6, 1e6)


CONFIGS = [
    # the configuration whose one GPU run after the gate|up fix faulted
    cw.make_config(2, 256, 4, 2, 128, 512, 1000, 8),
    small128(29, cw.CW_F32, 4, 2),
    small128(29, cw.CW_F16, 8, 2),
    small128(29, cw.CW_F32, 2, 2),
    small128(29, cw.CW_F16, 8, 1),
    cw.make_config(28, 1024, 16, 8, 128, 3072, 151936, 160, cw.CW_F32, 1e-6, 1e6),
    cw.make_config(36, 4096, 32, 8, 128, 12288, 151936, 4112, cw.CW_F16, 1e-6, 1e6),
]


@pytest.mark.parametrize("cfg", CONFIGS, ids=lambda c: f"L{c.n_layers}d{c.dim}h{c.n_heads}"
                         f"kv{c.n_kv_heads}t{c.kv_dtype}")
def test_model_layout_holds(cfg):
    rc, why = cw.step_layout_check(cfg, N_CU)
    assert rc == 0, why


@pytest.mark.parametrize("cfg", CONFIGS, ids=lambda c: f"L{c.n_layers}d{c.dim}h{c.n_heads}"
                         f"kv{c.n_kv_heads}t{c.kv_dtype}")
def test_split_gate_up_is_refused(cfg):
    """Gate and up as separate allocations: the gate|up phase reads 2*hidden
    rows of quants from the gate matrix, `hidden` rows past its end."""
    rc, why = cw.step_layout_check(cfg, N_CU, split_gate_up=True)
    assert rc == cw.CW_ERR_STATE, why
    nb = cfg.dim // 32
    past = cfg.hidden * nb * 16
    assert "layer 0 GATE|UP quants" in why, why
    assert f"({past} bytes past its end)" in why, why


def test_uncovered_shape_is_an_argument_error():
    cfg = cw.make_config(2, 64, 4, 2, 16, 128, 256, 12, cw.CW_F32, 1e-6, 1e6)
    rc, why = cw.step_layout_check(cfg, N_CU)
    assert rc == cw.CW_ERR_ARG
    assert "head_dim must be 128" in cw.lib().cw_last_error().decode()
