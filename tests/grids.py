"""Test helper: the IQ lattice tables as numpy arrays, read from the committed header, and the
reference shader text's copies when the reference checkout is present (never on the GPU box)."""
import os
import re

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "coachwhip_amd", "csrc", "cw_grids.h")
REF_METAL = "/root/reference/vendor/candle-metal-kernels/src/metal_src/quantized.metal"


def _parse_header():
    text = open(HEADER).read()
    out = {}
    for ctype, name, size, macro in re.findall(r"static const (\w+) cw_(\w+)\[(\d+)\] = \{(\w+)\};", text):
        body = re.search(r"#define %s \\(.*?)\n\n" % macro, text, re.S).group(1)
        vals = [int(v.rstrip("ul"), 16) for v in re.findall(r"0x[0-9a-f]+u?l*", body)]
        assert len(vals) == int(size)
        out[name] = np.array(vals, dtype=np.uint64 if ctype == "uint64_t" else np.uint32)
    return out


GRIDS = _parse_header()


def grid_bytes(name):
    """Each table entry as its little-endian bytes: (entries, 8) for u64 tables, (entries, 4) for u32."""
    g = GRIDS[name]
    return g.view(np.uint8).reshape(len(g), -1)


def ksigns_closed_form():
    i = np.arange(128)
    par = np.array([bin(v).count("1") & 1 for v in i])
    return (i | (par << 7)).astype(np.uint8)


def reference_table(name):
    """The table as written in the reference's shader text, or None without the checkout."""
    if not os.path.exists(REF_METAL):
        return None
    text = open(REF_METAL).read()
    m = re.search(r"GGML_TABLE_BEGIN\(\w+,\s*%s,\s*\w+\)(.*?)GGML_TABLE_END\(\)" % name, text, re.S)
    return [int(v, 0) for v in re.findall(r"0x[0-9a-fA-F]+|\b\d+\b", m.group(1))]


def reference_kvalues_iq4nl():
    """kvalues_iq4nl_f (quantized.metal:4561-4563) as written in the shader text, or None."""
    if not os.path.exists(REF_METAL):
        return None
    text = open(REF_METAL).read()
    m = re.search(r"kvalues_iq4nl_f\[16\]\s*=\s*\{(.*?)\}", text, re.S)
    return [float(v) for v in re.findall(r"-?\d+(?:\.\d*)?", m.group(1))]
