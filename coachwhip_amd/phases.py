"""Phase stamps of the one-launch decode layer (`k_moe_decode`) for configs 3 and 4.

Runs the library built with the stamps compiled in (`libcwmoe_phases.so`, made beside
`libcwmoe.so` by the package Makefile) and prints, per config, when the kernel's blocks reach each
of its eight points: start, routed, gate/up items done, at the barrier, arrived (the block's
hidden-row stores have landed), barrier open, hidden rows staged in LDS, end. Times are µs from
the earliest block's start in the same launch (thread 0 of each block reads s_memrealtime, a
100 MHz clock), over eager single-token calls synchronised between them, on a chain of 8 layers
of random experts so that no call finds its weights in a cache. Usage:

    python3 -m coachwhip_amd.phases [c3] [c4] [c4r16]

c4r16 is config 4 with its experts repacked in row groups of 16 (ExpertBank.rows16), whose
one-launch decode stages each pick's groups as K-split block items.
"""
import ctypes
import os
import statistics
import sys

import numpy as np

from . import _lib

POINTS = ["start", "routed", "gate/up done", "at the barrier", "arrived (stores landed)", "barrier open",
          "hidden rows staged", "end"]
CONFIGS = {
    # name: experts, top-k, hidden, expert FFN, formats, clamped SwiGLU with biases
    "c3": (256, 8, 2048, 512, ("IQ2_XXS", "IQ2_XXS", "IQ2_S"), False),
    "c4": (128, 4, 2880, 2880, ("MXFP4", "MXFP4", "MXFP4"), True),
    "c4r16": (128, 4, 2880, 2880, ("MXFP4", "MXFP4", "MXFP4"), True),
}
MAX_BLOCKS = 4096


def run(name, reps=4, layers=8, seed=5):
    import torch
    from . import formats as F
    from . import ops, synth
    lib = _lib.lib()
    E, K, H, I, fmts, act = CONFIGS[name]
    dts = tuple(getattr(F, f) for f in fmts)
    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev)
    gen.manual_seed(seed)
    shapes = [(I, H), (I, H), (H, I)]
    chain = []
    for _ in range(layers):
        banks = [ops.ExpertBank(synth.device_blocks(dts[m], E * shapes[m][0] * shapes[m][1], gen, dev), dts[m], shapes[m][0],
                                shapes[m][1], E, F.matrix_bytes(dts[m], *shapes[m])) for m in range(3)]
        ea = ops.ExpertAct.silu()
        if act:
            ea = ops.ExpertAct.clamped_swiglu(1.702, 7.0, *[torch.randn((E, n), generator=gen, device=dev) * 0.02 for n in (I, I, H)])
        if name.endswith("r16"):
            banks = [b.rows16() for b in banks]
        chain.append(ops.MoeLayer(*banks, n_experts=E, top_k=K, norm_topk_prob=True, act=ea))
    x = torch.randn((1, H), generator=gen, device=dev)
    buf = (ctypes.c_ulonglong * (MAX_BLOCKS * 8))()
    launches, nblk = [], None
    for rep in range(reps):
        for layer in chain:
            layer.forward(x, torch.randn((1, E), generator=gen, device=dev))
            torch.cuda.synchronize()
            if lib.cw_dbg_phases(buf, MAX_BLOCKS) != 0:
                raise RuntimeError("cw_dbg_phases failed")
            a = np.frombuffer(buf, dtype=np.uint64).reshape(MAX_BLOCKS, 8).astype(np.int64)
            if nblk is None:
                nblk = int(np.count_nonzero(a[:, 7]))
            if rep > 0:  # the first pass warms the chain up
                a = a[:nblk]
                launches.append((a - a[:, 0].min()) * 0.01)
    del chain
    torch.cuda.empty_cache()
    return nblk, launches


def table(name, nblk, launches, cus):
    r = np.concatenate(launches)
    out = ["%s: %d blocks, %d launches" % (name, nblk, len(launches)), "",
           "| point | median µs | 90th percentile | max |", "|---|---|---|---|"]
    for i, p in enumerate(POINTS):
        out.append("| %s | %.2f | %.2f | %.2f |" % (p, np.median(r[:, i]), np.percentile(r[:, i], 90), r[:, i].max()))
    med = lambda f: statistics.median([f(x) for x in launches])  # noqa: E731
    out.append("")
    out.append("Per launch (medians over the launches): last gate/up done %.2f µs, last at the barrier %.2f, last arrival %.2f, "
               "first block released %.2f, median release %.2f, last block ends %.2f." % (
                   med(lambda x: x[:, 2].max()), med(lambda x: x[:, 3].max()), med(lambda x: x[:, 4].max()),
                   med(lambda x: x[:, 5].min()), med(lambda x: np.median(x[:, 5])), med(lambda x: x[:, 7].max())))
    if nblk > cus:
        # blocks are placed in index order: block b is the (b // cus)-th on its CU
        for q in range((nblk + cus - 1) // cus):
            sel = np.concatenate([x[q * cus:(q + 1) * cus] for x in launches])
            out.append("Blocks placed %s on a CU (%d..%d): routed %.2f µs, gate/up done median %.2f and max %.2f, arrived median %.2f." % (
                ("first", "second", "third", "fourth")[min(q, 3)], q * cus, min(nblk, (q + 1) * cus) - 1, np.median(sel[:, 1]),
                np.median(sel[:, 2]), sel[:, 2].max(), np.median(sel[:, 4])))
    return "\n".join(out)


def main(argv):
    names = [a for a in argv if a in CONFIGS] or list(CONFIGS)
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libcwmoe_phases.so")
    if not os.path.exists(path):
        raise SystemExit("libcwmoe_phases.so is not built (make -C coachwhip_amd/csrc)")
    _lib.LIB_PATH = path
    import torch
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    for name in names:
        nblk, launches = run(name)
        print(table(name, nblk, launches, cus), flush=True)
        print(flush=True)


if __name__ == "__main__":
    main(sys.argv[1:])
