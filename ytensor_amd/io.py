"""yt::io on the device: YTensor's .yt checkpoint files loaded straight into
GPU memory and saved from it, through libythip's ythip_yt_* entry points
(include/ythip.h). The reading, inflating, type conversion and staging all run
in libythip.so (csrc/ytio.hip); this module only mirrors the reference's API.

Mirrors include/ytensor_io.hpp (namespace yt::io):
  compressMethod, verbose             module settings (ytensor_io.hpp:27-46)
  Closed / Read / Write / Append      file modes (ytensor_io.hpp:33-36)
  TensorInfo                          ytensor_io.hpp:67-78
  YTensorIO.open / close / getTensorNames / getTensorInfo / save / load /
  validateFile                        ytensor_io.hpp:81-180, src/ytensor_io.inl
  saveTensorBase / loadTensorBase     ytensor_io.hpp:182-198
Error behaviour follows the reference: open/save/close/loadTensorBase report
failure by returning False (load by returning None, where the reference's
load(tensor, name) returns false), getTensorInfo raises RuntimeError for an
unknown name, and messages go to stderr only when `verbose` is set. Tensors are
torch device tensors; load() converts on the way with the reference's casts
when asked for another float type.
"""
from __future__ import annotations

import ctypes
import os
import sys
from dataclasses import dataclass, field

import torch

from . import _lib

Closed, Read, Write, Append = 0, 1, 2, 3
compressMethod = ""  # "" (none) or "zlib"
verbose = False

# typeName <-> torch dtype for the dense types a device tensor can hold
_TORCH = {"float32": torch.float32, "bfloat16": torch.bfloat16, "float16": torch.float16,
          "float64": torch.float64, "int64": torch.int64, "int32": torch.int32, "int16": torch.int16,
          "int8": torch.int8, "uint8": torch.uint8, "bool": torch.bool}
_NAME = {v: k for k, v in _TORCH.items()}
_CODE = {torch.float32: _lib.F32, torch.float16: _lib.F16, torch.bfloat16: _lib.BF16}


def _warn(msg: str) -> None:
    if verbose:
        print(msg, file=sys.stderr)


@dataclass
class TensorInfo:
    """TensorInfo (include/ytensor_io.hpp:67-78); dataOffset is the payload's
    position in the file."""
    name: str
    typeName: str
    typeSize: int
    tensorType: str
    shape: list = field(default_factory=list)
    dataOffset: int = 0
    compressedSize: int = 0
    compressMethod: str = ""
    uncompressedSize: int = 0


def _info_of(h, i: int) -> TensorInfo:
    raw = _lib.YtTensorInfo()
    _lib.check(_lib.lib().ythip_yt_info(h, i, ctypes.byref(raw)), "ythip_yt_info")
    return TensorInfo(raw.name.decode(), raw.dtype.decode(), raw.type_size, raw.tensor_type.decode(),
                      [raw.shape[d] for d in range(raw.ndim)], raw.data_offset, raw.compressed_size,
                      raw.compress.decode(), raw.nbytes)


class YTensorIO:
    """yt::io::YTensorIO for device tensors."""

    def __init__(self):
        self._h = None          # read handle (Read mode, or the existing file in Write/Append)
        self._mode = Closed
        self._path = ""
        self._staged: list[tuple[str, torch.Tensor]] = []  # Write/Append: saved, written at close()
        self._disk: list[TensorInfo] = []

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    # ------------------------------------------------------------ open/close
    def open(self, fileName: str, fileMode: int = Read) -> bool:
        """YTensorIO::open (src/ytensor_io.inl:256-311)."""
        self.close()
        lib = _lib.lib()
        h = ctypes.c_void_p()
        st = lib.ythip_yt_open(os.fsencode(fileName), ctypes.byref(h))
        if fileMode in (Write, Append):
            # an existing, readable file contributes its tensors; anything else starts empty
            self._h = h if st == 0 else None
            self._disk = [_info_of(self._h, i) for i in range(lib.ythip_yt_count(self._h))] if self._h else []
            self._mode, self._path = fileMode, fileName
            return True
        if st != 0:
            _warn(f"Error: Failed to open file for reading: {fileName} ({lib.ythip_last_error().decode()})")
            return False
        self._h, self._mode, self._path = h, Read, fileName
        self._disk = [_info_of(h, i) for i in range(lib.ythip_yt_count(h))]
        return True

    def close(self) -> bool:
        """YTensorIO::close (src/ytensor_io.inl:313-417): Write/Append write the
        file now (one ythip_yt_save of every tensor saved since open)."""
        ok = True
        lib = _lib.lib() if self._mode != Closed else None
        if self._mode in (Write, Append):
            if self._h is not None:
                lib.ythip_yt_close(self._h)  # the writer reopens the existing file itself
                self._h = None
            keep = []  # torch tensors referenced by the descriptors until the call returns
            descs = (_lib.YtTensor * max(1, len(self._staged)))()
            for j, (name, t) in enumerate(self._staged):
                shape = (ctypes.c_int32 * max(1, t.dim()))(*t.shape)
                keep.append(shape)
                code = _CODE.get(t.dtype, _lib.YT_RAW)
                descs[j] = _lib.YtTensor(name.encode(), code, _NAME[t.dtype].encode(), t.element_size(), t.dim(),
                                         ctypes.cast(shape, ctypes.POINTER(ctypes.c_int32)),
                                         t.data_ptr() if t.numel() else None)
            stream = torch.cuda.current_stream().cuda_stream if torch.cuda.is_available() else None
            st = lib.ythip_yt_save(os.fsencode(self._path), len(self._staged), descs,
                                   compressMethod.encode(), int(self._mode == Append), stream)
            if st != 0:
                _warn(f"Error: Failed to write {self._path}: {lib.ythip_last_error().decode()}")
                ok = False
        elif self._h is not None:
            lib.ythip_yt_close(self._h)
        self._h, self._mode, self._path, self._staged, self._disk = None, Closed, "", [], []
        return ok

    # ------------------------------------------------------------ queries
    def _names(self) -> list[str]:
        names = [i.name for i in self._disk]
        for n, _ in self._staged:
            if n not in names:
                names.append(n)
        return names

    def getTensorNames(self) -> list[str]:
        """getTensorNames (src/ytensor_io.inl:419-425)."""
        return self._names()

    def getTensorInfo(self, name: str = "") -> TensorInfo:
        """getTensorInfo (src/ytensor_io.inl:427-443): "" is the first tensor;
        RuntimeError when there is none of that name."""
        staged = dict(self._staged)
        names = self._names()
        if not names:
            raise RuntimeError("No tensors available")
        key = names[0] if name == "" else name
        if key in staged:
            t = staged[key]
            nb = t.numel() * t.element_size()
            return TensorInfo(key, _NAME[t.dtype], t.element_size(), "dense", list(t.shape), 0, nb,
                              compressMethod, nb)
        for i in self._disk:
            if i.name == key:
                return i
        raise RuntimeError("Tensor not found: " + name)

    def validateFile(self) -> bool:
        """validateFile (src/ytensor_io.inl:445-456): an open file with the magic."""
        return self._mode != Closed and self._h is not None

    # ------------------------------------------------------------ save/load
    def save(self, tensor: torch.Tensor, name: str = "") -> bool:
        """YTensorIO::save (src/ytensor_io.inl:703-783): snapshot of the tensor
        (the reference clones it), written at close(); "" names it by position,
        an existing name is replaced in place."""
        if self._mode not in (Write, Append):
            _warn("Error: File not open for writing")
            return False
        if tensor.dtype not in _NAME:
            _warn(f"Error: dtype {tensor.dtype} has no YTensor type name")
            return False
        if not tensor.is_cuda:
            _warn("Error: save() takes device tensors")
            return False
        name = name if name else str(len(self._names()))
        snap = tensor.detach().contiguous().clone()
        for j, (n, _) in enumerate(self._staged):
            if n == name:
                self._staged[j] = (name, snap)
                return True
        self._staged.append((name, snap))
        return True

    def load(self, name: str = "", dtype: torch.dtype | None = None, out: torch.Tensor | None = None,
             device: torch.device | str | None = None, sync: bool = True) -> torch.Tensor | None:
        """YTensorIO::load (src/ytensor_io.inl:785-830) into device memory.

        dtype None keeps the stored type (the bytes are copied unchanged);
        torch.float32 / bfloat16 / float16 convert with the reference's casts.
        `out` (contiguous, on the device) receives the data in place of a new
        tensor. Returns None when the reference's load would return false."""
        try:
            info = self.getTensorInfo(name)
        except RuntimeError as exc:
            _warn(f"Error: {exc}")
            return None
        staged = dict(self._staged)
        if info.name in staged:  # saved in this session, not written yet
            t = staged[info.name]
            if dtype is not None and dtype != t.dtype:
                _warn("Error: type conversion of a tensor not yet written is not supported")
                return None
            return t.clone() if out is None else out.copy_(t)
        if info.tensorType != "dense":
            _warn(f"Error: tensor '{info.name}' is '{info.tensorType}'; only dense tensors load to the device")
            return None
        if dtype is None:
            if info.typeName not in _TORCH:
                _warn(f"Error: type '{info.typeName}' has no device counterpart")
                return None
            tdt, code = _TORCH[info.typeName], _lib.YT_RAW
        elif dtype in _CODE:
            tdt, code = dtype, _CODE[dtype]
        else:
            _warn(f"Error: conversion to {dtype} is not supported")
            return None
        shape = tuple(info.shape)
        if out is None:
            dev = torch.device(device) if device is not None else torch.device("cuda", torch.cuda.current_device())
            out = torch.empty(shape, dtype=tdt, device=dev)
        elif not (out.is_cuda and out.is_contiguous() and out.dtype == tdt and out.numel() == _numel(shape)):
            raise ValueError(f"load: out must be a contiguous {tdt} device tensor of {_numel(shape)} elements")
        lib = _lib.lib()
        idx = lib.ythip_yt_find(self._h, info.name.encode())
        if idx < 0:
            return None
        with torch.cuda.device(out.device):
            stream = torch.cuda.current_stream().cuda_stream
            st = lib.ythip_yt_load(self._h, idx, out.data_ptr() if out.numel() else None, code,
                                   out.numel() * out.element_size(), stream)
            if st != 0:
                _warn(f"Error: {lib.ythip_last_error().decode()}")
                if st > 0:  # a HIP error is not a file problem: surface it
                    _lib.check(st, "ythip_yt_load")
                return None
            if sync:
                torch.cuda.current_stream().synchronize()
        return out

    def load_many(self, items) -> None:
        """Loads several tensors into given device views with one C call and
        one final wait: items = [(name, out_tensor), ...]; every out must be
        contiguous and of the stored size, its dtype picks the conversion
        (the stored type = bytes copied unchanged). Raises RuntimeError naming
        the problem; nothing is queued unless every item is valid."""
        lib = _lib.lib()
        if self._h is None:
            raise RuntimeError("load_many: no file open for reading")
        pos: dict = {}
        for k, i in enumerate(self._disk):
            pos.setdefault(i.name, k)  # the first of a repeated name, as ythip_yt_find
        n = len(items)
        idx = (ctypes.c_int * max(1, n))()
        dsts = (ctypes.c_void_p * max(1, n))()
        codes = (ctypes.c_int * max(1, n))()
        sizes = (ctypes.c_uint64 * max(1, n))()
        dev = None
        for j, (name, out) in enumerate(items):
            if name not in pos:
                raise RuntimeError(f"load_many: tensor not found: {name}")
            info = self._disk[pos[name]]
            if _TORCH.get(info.typeName) == out.dtype:
                code = _lib.YT_RAW
            elif out.dtype in _CODE:
                code = _CODE[out.dtype]
            else:
                raise RuntimeError(f"load_many: '{name}' is {info.typeName}; no conversion to {out.dtype}")
            if not (out.is_cuda and out.is_contiguous() and out.numel() == _numel(info.shape)):
                raise RuntimeError(f"load_many: '{name}' has shape {info.shape}, the destination {tuple(out.shape)}")
            if dev is None:
                dev = out.device
            elif out.device != dev:
                raise RuntimeError("load_many: all destinations must be on one device")
            idx[j], codes[j] = pos[name], code
            dsts[j] = out.data_ptr() if out.numel() else None
            sizes[j] = out.numel() * out.element_size()
        if n == 0:
            return
        with torch.cuda.device(dev):
            st = lib.ythip_yt_load_many(self._h, n, idx, dsts, codes, sizes, torch.cuda.current_stream().cuda_stream)
            if st != 0:
                raise RuntimeError(f"ythip_yt_load_many failed ({st}): {lib.ythip_last_error().decode()}")
            _lib.check(lib.ythip_yt_sync(self._h), "ythip_yt_sync")


def _numel(shape) -> int:
    n = 1
    for d in shape:
        n *= int(d)
    return n


def saveTensorBase(fileName: str, tensor: torch.Tensor, name: str = "") -> bool:
    """saveTensorBase (src/ytensor_io.inl:832-842)."""
    io = YTensorIO()
    if not io.open(fileName, Write):
        return False
    if not io.save(tensor, name):
        return False
    return io.close()


def loadTensorBase(fileName: str, name: str = "", dtype: torch.dtype | None = None) -> torch.Tensor | None:
    """loadTensorBase (src/ytensor_io.inl:844-850)."""
    io = YTensorIO()
    if not io.open(fileName, Read):
        return None
    try:
        return io.load(name, dtype)
    finally:
        io.close()
