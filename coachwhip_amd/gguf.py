"""GGUF files through the library's reader (cw_gguf_* in include/cwmoe.h).

The reader follows candle's ``Content::read`` (vendor/candle-core/src/quantized/gguf_file.rs:
469-567) and also accepts IQ3_S and IQ2_S. ``moe_layer`` turns a layer's expert tensors
(``blk.{l}.ffn_{gate,up,down}_exps.weight``, laid out as ExpertStore::new reads them,
crates/engine/src/experts.rs:697-718) and its router (``ffn_gate_inp``) into a ``MoeLayer`` and
router weight on the device.
"""
import ctypes

import numpy as np
import torch

from . import ops
from ._lib import CwError, check, lib, CW_EINVAL

GGUF_F32, GGUF_F16 = 0, 1
SWIGLU_ALPHA, SWIGLU_LIMIT = 1.702, 7.0   # crates/engine/src/model_gptoss.rs:16-17
PARTS = ("gate", "up", "down")


class GGUFFile:
    """An open GGUF file; tensor bytes are views of its read-only mapping (valid until close)."""

    def __init__(self, path):
        self._h = lib().cw_gguf_open(str(path).encode())
        if not self._h:
            raise CwError(CW_EINVAL, lib().cw_last_error().decode(errors="replace"))
        self.path = str(path)

    def close(self):
        if self._h:
            lib().cw_gguf_close(self._h)
            self._h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:  # interpreter shutdown: the library may already be gone
            pass

    @property
    def version(self) -> int:
        return lib().cw_gguf_version(self._h)

    def __len__(self) -> int:
        return lib().cw_gguf_n_tensors(self._h)

    def find(self, name: str) -> int:
        return lib().cw_gguf_find(self._h, name.encode())

    def tensor(self, i: int):
        """(name, GGUF type id, dims outermost first, file offset, bytes)."""
        name = ctypes.c_char_p()
        dtype, nd = ctypes.c_int(), ctypes.c_int()
        dims = (ctypes.c_int64 * 4)()
        off, nbytes = ctypes.c_int64(), ctypes.c_int64()
        check(lib().cw_gguf_tensor(self._h, i, ctypes.byref(name), ctypes.byref(dtype), ctypes.byref(nd), dims,
                                   ctypes.byref(off), ctypes.byref(nbytes)))
        return name.value.decode(), dtype.value, tuple(dims[:nd.value]), off.value, nbytes.value

    def names(self):
        return [self.tensor(i)[0] for i in range(len(self))]

    def data(self, i: int) -> np.ndarray:
        """The bytes of tensor i (a read-only view of the mapping)."""
        nbytes = self.tensor(i)[4]
        ptr = lib().cw_gguf_data(self._h, i)
        if not ptr:
            raise CwError(CW_EINVAL, "gguf: no data for tensor %d" % i)
        return np.ctypeslib.as_array((ctypes.c_uint8 * nbytes).from_address(ptr))

    def meta_int(self, key: str):
        v = ctypes.c_int64()
        check(lib().cw_gguf_meta_int(self._h, key.encode(), ctypes.byref(v)))
        return v.value

    def meta_float(self, key: str):
        v = ctypes.c_double()
        check(lib().cw_gguf_meta_float(self._h, key.encode(), ctypes.byref(v)))
        return v.value

    def meta_str(self, key: str):
        v = lib().cw_gguf_meta_str(self._h, key.encode())
        return None if v is None else v.decode(errors="replace")

    def experts(self, layer: int, which: int):
        """(GGUF type, n_experts, n, k, expert_bytes, bytes of all experts) of one expert tensor."""
        dtype, ne, n, k, eb = ctypes.c_int(), ctypes.c_int64(), ctypes.c_int64(), ctypes.c_int64(), ctypes.c_int64()
        ptr = ctypes.c_void_p()
        check(lib().cw_gguf_experts(self._h, layer, which, ctypes.byref(dtype), ctypes.byref(ne), ctypes.byref(n),
                                    ctypes.byref(k), ctypes.byref(eb), ctypes.byref(ptr)))
        raw = np.ctypeslib.as_array((ctypes.c_uint8 * (ne.value * eb.value)).from_address(ptr.value))
        return dtype.value, ne.value, n.value, k.value, eb.value, raw

    def bank(self, layer: int, n_slots: int, device="cuda", shrink=(False, False, False)):
        """A device bank of n_slots slots for the layer's experts, with the experts' bytes copied
        once into pinned host memory as the bank's source (the host-memory expert store); matrices
        with shrink[m] are held as Q2_K."""
        from .bank import Bank, pinned_copy
        host, dtypes, shapes, counts = [], [], [], set()
        for which in range(3):
            dtype, ne, n, k, eb, raw = self.experts(layer, which)
            host.append(pinned_copy(raw))
            dtypes.append(dtype)
            shapes.append((n, k))
            counts.add(ne)
        if len(counts) != 1:
            raise CwError(CW_EINVAL, "gguf: layer %d has differing expert counts" % layer)
        return Bank(host, dtypes, shapes, counts.pop(), n_slots, device, shrink=shrink)

    def _dense(self, name, device):
        """A F32 or F16 tensor by name as an f32 device tensor (outermost dim first), or None."""
        i = self.find(name)
        if i < 0:
            return None
        _, dtype, dims, _, _ = self.tensor(i)
        if dtype not in (GGUF_F32, GGUF_F16):
            raise CwError(CW_EINVAL, "gguf: %s is type %d (f32 or f16 expected)" % (name, dtype))
        a = np.array(self.data(i)).view(np.float32 if dtype == GGUF_F32 else np.float16).reshape(dims)
        return torch.from_numpy(a.astype(np.float32)).to(device)

    def moe_layer(self, layer: int, top_k: int, norm_topk_prob: bool = True, device="cuda"):
        """(MoeLayer with the layer's experts resident on the device, router weight (E, h) f32 on
        the device or None, router bias or None).

        With ``ffn_{gate,up,down}_exps.bias`` present (gpt-oss) the activation is the clamped
        SwiGLU with those biases (alpha 1.702, limit 7), and a down matrix wider than the
        intermediate size sets the padding; the router is zero-padded to the experts' input
        width, as crates/engine/src/model_gptoss.rs:141-175 loads it."""
        p = "blk.%d." % layer
        banks = []
        for which in range(3):
            dtype, ne, n, k, eb, raw = self.experts(layer, which)
            banks.append(ops.ExpertBank(ops.to_device(np.array(raw), device), dtype, n, k, ne, eb))
        gate, up, down = banks
        if not (gate.n_slots == up.n_slots == down.n_slots) or (gate.n, gate.k) != (up.n, up.k) or down.n != gate.k \
                or down.k < gate.n:
            raise CwError(CW_EINVAL, "gguf: layer %d expert tensors do not fit together" % layer)
        biases = [self._dense(p + "ffn_%s_exps.bias" % m, device) for m in PARTS]
        act = None
        if any(b is not None for b in biases):
            if any(b is None for b in biases):
                raise CwError(CW_EINVAL, "gguf: layer %d has only some expert biases" % layer)
            act = ops.ExpertAct.clamped_swiglu(SWIGLU_ALPHA, SWIGLU_LIMIT, *biases,
                                               pad=down.k if down.k > gate.n else 0)
        layer_moe = ops.MoeLayer(gate, up, down, gate.n_slots, top_k, norm_topk_prob, act=act)
        router = self._dense(p + "ffn_gate_inp.weight", device)
        bias = self._dense(p + "ffn_gate_inp.bias", device)
        if router is not None:
            if router.dim() != 2 or router.shape[1] > gate.k:
                raise CwError(CW_EINVAL, "gguf: router of layer %d is %s" % (layer, tuple(router.shape)))
            if router.shape[1] < gate.k:
                router = torch.nn.functional.pad(router, (0, gate.k - router.shape[1])).contiguous()
        return layer_moe, router, bias
