"""Write the fused decode step's buffer plan (cw_step_dry_plan) for the CPU
execution in step_emu.cpp: four u64 (argument block bytes, layer table
bytes, allocation count, layer record bytes), the argument block, the layer
table, then the allocations' addresses and sizes (u64 each).

The argument block is the plan's last allocation and the layer table the
allocation its first pointer names, so both record sizes come from the plan
itself; step_emu checks them against its own build of the structures."""
import ctypes as C
import struct

import numpy as np

import cw

ARGS_MAX, LAYER_MAX, EXT_MAX = 4096, 1 << 20, 4096


def write_plan(cfg, n_cu, path, split_gate_up=False):
    args = np.zeros(ARGS_MAX, np.uint8)
    layers = np.zeros(LAYER_MAX, np.uint8)
    ext_p = (C.c_void_p * EXT_MAX)()
    ext_b = np.zeros(EXT_MAX, np.uint64)
    n = C.c_int()
    cw.check(cw.lib().cw_step_dry_plan(C.byref(cfg), n_cu, 1 if split_gate_up else 0,
                                       args.ctypes.data, ARGS_MAX, layers.ctypes.data, LAYER_MAX,
                                       C.cast(ext_p, C.c_void_p), ext_b.ctypes.data, EXT_MAX,
                                       C.byref(n)))
    ptrs = np.array([ext_p[i] or 0 for i in range(n.value)], np.uint64)
    sizes = ext_b[:n.value]
    args_bytes = int(sizes[-1])
    table = int(args[:8].view(np.uint64)[0])
    layer_total = int(sizes[int(np.nonzero(ptrs == table)[0][0])])
    with open(path, "wb") as f:
        f.write(struct.pack("<4Q", args_bytes, layer_total, n.value, layer_total // cfg.n_layers))
        f.write(args[:args_bytes].tobytes())
        f.write(layers[:layer_total].tobytes())
        f.write(ptrs.tobytes())
        f.write(sizes.tobytes())
    return n.value
