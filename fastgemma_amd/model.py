"""The .fgm model on the GPU: Python mirror of crates/fgm-core/src/model.rs
(Model, QLinear) and of the weight selection in forward.rs:26-89 (DualW,
WeightSel), over the C ABI in include/fgm_hip.h (fgm_hip_model_*).

The native library maps the file, parses the header and, with
``resident=True``, copies the tensor body to HBM once; tensors are then handed
out as views of the mapping (numpy) and, when resident, as device addresses.
"""
from __future__ import annotations

import ctypes as C
import enum
import json
import os
from dataclasses import dataclass

import numpy as np

from . import FgmHipError, LinearInfo, TensorInfo, check, lib


class WeightSel(enum.Enum):
    """Which weight a GEMM uses, as a row-count threshold (forward.rs:45-69)."""
    Lo = 0      # always the file's primary (int4 where the converter wrote int4)
    Hi = 1      # always the int8 twin where one exists
    Above = 2   # the int8 twin once a GEMM has at least `threshold` rows


@dataclass(frozen=True)
class Selection:
    sel: WeightSel
    threshold: int = 16

    @staticmethod
    def parse(value: str | None) -> "Selection":
        """FGM_WEIGHTS=int4|int8|auto[:M], default auto:16 (forward.rs:58-69)."""
        t = C.c_int(16)
        s = lib().fgm_hip_weight_sel(None if value is None else value.encode(), C.byref(t))
        return Selection(WeightSel(s), t.value)

    @staticmethod
    def from_env() -> "Selection":
        return Selection.parse(os.environ.get("FGM_WEIGHTS"))


@dataclass
class QLinear:
    """A quantised linear weight (model.rs:104-117): geometry, the blobs as
    views of the mapping, and their device addresses when resident."""
    name: str
    bits: int
    n: int
    k: int
    group: int
    hadamard: int
    info: LinearInfo

    def blob(self) -> np.ndarray:
        nbytes = self.n * self.k // 2 if self.bits == 4 else self.n * self.k
        dt = np.uint8 if self.bits == 4 else np.int8
        return np.ctypeslib.as_array(C.cast(self.info.b_host, C.POINTER(C.c_byte)), (nbytes,)).view(dt)

    def scales(self) -> np.ndarray:
        if self.bits == 4:
            cnt = (self.k // self.group) * self.n
            return np.ctypeslib.as_array(C.cast(self.info.b_scale_host, C.POINTER(C.c_uint16)), (cnt,))
        return np.ctypeslib.as_array(C.cast(self.info.b_scale_host, C.POINTER(C.c_float)), (self.n,))


class Model:
    """A .fgm file (model.rs:119-213)."""

    def __init__(self, path: str, resident: bool = False):
        self._h = lib().fgm_hip_model_open(os.fsencode(path), 1 if resident else 0)
        if not self._h:
            raise FgmHipError(lib().fgm_hip_last_error().decode())
        self.resident = resident
        self.cfg = json.loads(lib().fgm_hip_model_config(self._h).decode())
        self.meta = json.loads(lib().fgm_hip_model_meta(self._h).decode())

    def close(self) -> None:
        if self._h:
            lib().fgm_hip_model_close(self._h)
            self._h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def has(self, name: str) -> bool:
        return bool(lib().fgm_hip_model_has(self._h, name.encode()))

    def names(self) -> list[str]:
        n = lib().fgm_hip_model_tensor_count(self._h)
        return [lib().fgm_hip_model_tensor_name(self._h, i).decode() for i in range(n)]

    def tensor(self, name: str) -> TensorInfo:
        t = TensorInfo()
        check(lib().fgm_hip_model_tensor(self._h, name.encode(), C.byref(t)))
        return t

    def shape(self, name: str) -> list[int]:
        t = self.tensor(name)
        return [int(t.shape[i]) for i in range(t.ndim)]

    def _view(self, name: str, dtype) -> np.ndarray:
        t = self.tensor(name)
        raw = np.ctypeslib.as_array(C.cast(t.host, C.POINTER(C.c_ubyte)), (t.nbytes,))
        return raw.view(dtype)

    def f32s(self, name: str) -> np.ndarray:
        return self._view(name, np.float32)

    def f16s(self, name: str) -> np.ndarray:
        return self._view(name, np.uint16)

    def i8s(self, name: str) -> np.ndarray:
        return self._view(name, np.int8)

    def u8s(self, name: str) -> np.ndarray:
        return self._view(name, np.uint8)

    def total_bytes(self) -> int:
        return int(lib().fgm_hip_model_total_bytes(self._h))

    def _linear(self, info: LinearInfo, name: str) -> QLinear:
        return QLinear(name, info.bits, info.n, info.k, info.group, info.hadamard, info)

    def linear(self, name: str) -> QLinear:
        """model.rs:167-192: q4g (f16 scales, meta.group default 64) or q8c."""
        info = LinearInfo()
        check(lib().fgm_hip_model_linear(self._h, name.encode(), C.byref(info)))
        return self._linear(info, name)

    def dual(self, name: str) -> "DualW":
        """The linear and its int8 twin `<name>.i8` when the file has one
        (model.rs:194-201)."""
        return DualW(self, name)

    def gather(self, name: str, rows, out=None):
        """Rows of a q8r / q4r table on the GPU (model.rs:203-213); `rows`
        and `out` are GPU tensors (int32 [count], float32 [count, k])."""
        check(lib().fgm_hip_model_gather_dev(self._h, name.encode(), rows.data_ptr(), rows.numel(),
                                             out.data_ptr(), _stream()))
        return out


class DualW:
    """A weight the file may carry in two quantisations (forward.rs:26-89)."""

    def __init__(self, model: Model, name: str):
        self.model, self.name = model, name

    def has_hi(self) -> bool:
        return self.model.has(self.name + ".i8")

    def pick(self, m: int, sel: Selection) -> QLinear:
        """DualW::pick (forward.rs:74-81), resolved by the library."""
        info = LinearInfo()
        check(lib().fgm_hip_model_dual(self.model._h, self.name.encode(), m, sel.sel.value,
                                       sel.threshold, C.byref(info)))
        alt = self.name + ".i8"
        hi = self.has_hi() and info.b_host == self.model.linear(alt).info.b_host
        return self.model._linear(info, alt if hi else self.name)


def _stream():
    import torch
    return torch.cuda.current_stream().cuda_stream


def linear_run(w: QLinear, a, m: int, lda: int, out, scratch=None) -> None:
    """Gemm::run (forward.rs:140-158) on a resident weight: out[m][0..n) =
    w . a[m][0..k) with FWHT of w.hadamard, per-row int8 quantisation and the
    GEMM.  `a`, `out`: GPU float32 tensors."""
    import torch
    nb = lib().fgm_hip_linear_scratch_bytes(m, w.k)
    sc = scratch if scratch is not None else torch.empty(max(nb, 1), dtype=torch.uint8, device=a.device)
    check(lib().fgm_hip_linear_run_dev(C.byref(w.info), a.data_ptr(), m, lda, out.data_ptr(),
                                       sc.data_ptr(), nb, _stream()))
    out._fgm_keep = sc
