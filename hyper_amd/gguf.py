"""GGUF expert loading through libhymoe's reader (include/hymoe.h, hy_gguf_*): the names and behaviour of the
reference's `GGUF` class (src/gguf.h:38-70, src/gguf.cpp:84-285) and `expert_tensors` (src/experts.cu:12-22).

The file is memory-mapped by the library; tensor views here are zero-copy numpy arrays over that mapping and stay
valid while the GGUF object is open.  `expert_layer` turns one layer's expert tensors into an `ExpertLayer`, which
`moe.MoeDev` / `moe.upload_experts` (or the C ABI's `hy_upload_experts`) place on the device.
"""
import ctypes
import warnings
from dataclasses import dataclass
from typing import Dict, List, Optional, Tuple

import numpy as np
import torch

from . import check, hy_expert_tensors, hy_gguf_tensor_info, lib
from .formats import ExpertLayer, GType, row_bytes


@dataclass
class GTensor:
    """A tensor of the file (src/gguf.h:22-32): ne in ggml order (ne[0] = row length), data as uint8 bytes."""
    name: str
    type: int
    ne: Tuple[int, ...]
    nbytes: int
    ptr: int
    owner: object = None   # the GGUF whose mapping holds the bytes

    def data(self) -> np.ndarray:
        """The tensor's bytes, a read-only view of the mapping.  The view keeps the GGUF object alive; it must not be
        used after an explicit close()."""
        buf = (ctypes.c_uint8 * self.nbytes).from_address(self.ptr)
        buf.owner = self.owner
        a = np.frombuffer(buf, dtype=np.uint8)
        a.flags.writeable = False
        return a

    def rows(self) -> int:
        n = 1
        for x in self.ne[1:]:
            n *= x
        return n


def _tensor(info: hy_gguf_tensor_info, owner) -> GTensor:
    return GTensor(info.name.decode(errors="replace"), int(info.type), tuple(int(info.ne[d]) for d in range(info.n_dims)),
                   int(info.nbytes), int(info.data or 0), owner)


class GGUF:
    """A read-only GGUF v2/v3 file (or the shards of a split model, given the first: <name>-00001-of-0000N.gguf)."""

    def __init__(self, path: str):
        h = ctypes.c_void_p()
        check(lib().hy_gguf_open(str(path).encode(), ctypes.byref(h)))
        self._h = h

    def close(self) -> None:
        if getattr(self, "_h", None) is not None and self._h.value:
            lib().hy_gguf_close(self._h)
            self._h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    # ---- metadata (GGUF::has / get_int / get_float / get_str / get_int_arr / get_float_arr)
    def arch(self) -> str:
        return lib().hy_gguf_arch(self._h).decode()

    def has(self, key: str) -> bool:
        return bool(lib().hy_gguf_has(self._h, key.encode()))

    def get_int(self, key: str, default: Optional[int] = None) -> int:
        if default is not None and not self.has(key):
            return default
        v = ctypes.c_int64()
        check(lib().hy_gguf_get_int(self._h, key.encode(), ctypes.byref(v)))
        return v.value

    def get_float(self, key: str, default: Optional[float] = None) -> float:
        if default is not None and not self.has(key):
            return default
        v = ctypes.c_double()
        check(lib().hy_gguf_get_float(self._h, key.encode(), ctypes.byref(v)))
        return v.value

    def get_str(self, key: str) -> str:
        v = ctypes.c_char_p()
        check(lib().hy_gguf_get_str(self._h, key.encode(), ctypes.byref(v)))
        return v.value.decode()

    def _arr(self, fn, key: str, ctype) -> list:
        n = ctypes.c_size_t()
        check(fn(self._h, key.encode(), None, 0, ctypes.byref(n)))
        buf = (ctype * max(n.value, 1))()
        check(fn(self._h, key.encode(), buf, n.value, ctypes.byref(n)))
        return list(buf[:n.value])

    def get_int_arr(self, key: str) -> List[int]:
        return self._arr(lib().hy_gguf_get_int_arr, key, ctypes.c_int64)

    def get_float_arr(self, key: str) -> List[float]:
        return self._arr(lib().hy_gguf_get_float_arr, key, ctypes.c_double)

    # ---- tensors (GGUF::tensors / tensor / need)
    def tensors(self) -> Dict[str, GTensor]:
        out = {}
        for i in range(lib().hy_gguf_n_tensors(self._h)):
            info = hy_gguf_tensor_info()
            check(lib().hy_gguf_tensor_at(self._h, i, ctypes.byref(info)))
            t = _tensor(info, self)
            out[t.name] = t
        return out

    def tensor(self, name: str) -> Optional[GTensor]:
        """The tensor, or None if the file has none of that name."""
        info = hy_gguf_tensor_info()
        if lib().hy_gguf_tensor(self._h, name.encode(), ctypes.byref(info)) != 0:
            return None
        return _tensor(info, self)

    def need(self, name: str) -> GTensor:
        info = hy_gguf_tensor_info()
        check(lib().hy_gguf_tensor(self._h, name.encode(), ctypes.byref(info)))
        return _tensor(info, self)

    def expert_tensors(self, il: int, E: int) -> hy_expert_tensors:
        """blk.<il>.ffn_{gate,up,down}_exps.weight of E experts, as the C ABI's hy_expert_tensors
        (host pointers into the mapping; ready for hy_upload_experts)."""
        t = hy_expert_tensors()
        check(lib().hy_gguf_expert_tensors(self._h, il, E, ctypes.byref(t)))
        return t


def expert_layer(g: GGUF, il: int, E: Optional[int] = None, clamp: float = 0.0) -> ExpertLayer:
    """Layer il's experts as an ExpertLayer over the file's bytes (host, zero-copy).  gate/up ne = [d, ff, E] and
    down ne = [ff, d, E] (tools/cpumoebench.cu:89-91); E defaults to the tensors' third dimension."""
    gt = g.need(f"blk.{il}.ffn_gate_exps.weight")
    dt = g.need(f"blk.{il}.ffn_down_exps.weight")
    if E is None:
        E = gt.ne[2] if len(gt.ne) > 2 else 1
    t = g.expert_tensors(il, E)
    n, ff = gt.ne[0], gt.ne[1]
    if dt.ne[0] != ff or dt.ne[1] != n:
        raise ValueError(f"layer {il}: down shape {dt.ne} does not match gate/up [{n}, {ff}]")
    tg, td = GType(t.tg), GType(t.td)
    if t.gb != ff * row_bytes(tg, n) or t.db != n * row_bytes(td, ff):
        raise ValueError(f"layer {il}: {E} experts do not fit the tensors' sizes")
    up = g.need(f"blk.{il}.ffn_up_exps.weight")

    def view(tt: GTensor, rows: int, rb: int) -> torch.Tensor:
        # read-only bytes of the mapping (torch warns that it cannot mark the tensor read-only; nothing writes it)
        with warnings.catch_warnings():
            warnings.simplefilter("ignore", UserWarning)
            return torch.from_numpy(tt.data()[: E * rows * rb].reshape(E, rows, rb))

    return ExpertLayer(tg, td, E, ff, n, view(gt, ff, row_bytes(tg, n)), view(up, ff, row_bytes(tg, n)),
                       view(dt, n, row_bytes(td, ff)), clamp)
