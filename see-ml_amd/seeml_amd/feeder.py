"""Python view of the native batch feeder (see-ml_amd/csrc/feeder.cc).

Mirrors the reference's Dataset (runtime/feeder/dataset.h:39-177): same
constructors, serving order, shuffle, serving-position snapshots, split and
.sds files. Everything runs in the backend library (host code); errors raise
RuntimeError with the reference's "Dataset: <message>" text.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from . import _lib


def _ptr(a: np.ndarray):
    return C.c_void_p(a.ctypes.data) if a is not None and a.size else C.c_void_p(0)


class Dataset:
    def __init__(self, handle):
        self._L = _lib.lib()
        self._h = handle

    def __del__(self):
        h, self._h = getattr(self, "_h", None), None
        if h:
            self._L.seeml_hip_dataset_free(h)

    @staticmethod
    def _make(fn, *args) -> "Dataset":
        L = _lib.lib()
        out = C.c_void_p()
        err = C.create_string_buffer(512)
        if getattr(L, fn)(*args, C.byref(out), err, 512) != 0:
            raise RuntimeError(err.value.decode())
        return Dataset(out)

    @staticmethod
    def from_tokens(tokens, num_records: int, seq: int) -> "Dataset":
        t = np.ascontiguousarray(tokens, np.int32)
        return Dataset._make("seeml_hip_dataset_from_tokens", _ptr(t), t.size, num_records, seq)

    @staticmethod
    def from_memory(inputs, labels, num_samples: int, input_dim: int, label_kind: int,
                    label_dim: int = 0) -> "Dataset":
        x = np.ascontiguousarray(inputs, np.float32).reshape(-1)
        lab = np.frombuffer(bytes(labels), np.uint8) if labels is not None else np.zeros(0, np.uint8)
        return Dataset._make("seeml_hip_dataset_from_memory", _ptr(x), x.size, _ptr(lab), lab.size,
                             num_samples, input_dim, label_kind, label_dim)

    @staticmethod
    def load(path: str) -> "Dataset":
        return Dataset._make("seeml_hip_dataset_load", path.encode())

    def _check(self, rc: int):
        if rc != 0:
            raise RuntimeError(self._L.seeml_hip_dataset_error(self._h).decode())

    def save(self, path: str):
        self._check(self._L.seeml_hip_dataset_save(self._h, path.encode()))

    @property
    def num_samples(self) -> int:
        return self._L.seeml_hip_dataset_num_samples(self._h)

    @property
    def input_dim(self) -> int:
        return self._L.seeml_hip_dataset_input_dim(self._h)

    @property
    def label_kind(self) -> int:
        return self._L.seeml_hip_dataset_label_kind(self._h)

    @property
    def input_kind(self) -> int:
        return self._L.seeml_hip_dataset_input_kind(self._h)

    def label_bytes_per_sample(self) -> int:
        return self._L.seeml_hip_dataset_label_bytes_per_sample(self._h)

    def validate_class_labels(self, num_classes: int):
        self._check(self._L.seeml_hip_dataset_validate_class_labels(self._h, num_classes))

    def fill_batch(self, batch: int, labels: bool = True):
        """The next `batch` rows as (inputs, label bytes): inputs are int32
        token ids for token corpora, float32 rows otherwise."""
        if self.input_kind == 1:
            x = np.zeros(batch, np.int32)
            lab = np.zeros(batch * 4, np.uint8) if labels else None
        else:
            x = np.zeros(batch * self.input_dim, np.float32)
            lb = self.label_bytes_per_sample()
            lab = np.zeros(batch * lb, np.uint8) if labels and lb else None
        self._L.seeml_hip_dataset_fill_batch(self._h, batch, _ptr(x), _ptr(lab) if lab is not None else None)
        return x, (lab.tobytes() if lab is not None else b"")

    def rewind(self):
        self._L.seeml_hip_dataset_rewind(self._h)

    def enable_shuffle(self, seed: int):
        self._L.seeml_hip_dataset_enable_shuffle(self._h, seed)

    def serving_pos(self) -> tuple[int, int]:
        c, e = C.c_uint64(), C.c_uint64()
        self._L.seeml_hip_dataset_get_serving_pos(self._h, C.byref(c), C.byref(e))
        return c.value, e.value

    def restore_serving_pos(self, cursor: int, epoch: int):
        self._L.seeml_hip_dataset_restore_serving_pos(self._h, cursor, epoch)

    def skip_served(self, rows: int):
        self._check(self._L.seeml_hip_dataset_skip_served(self._h, rows))

    def split_validation(self, fraction: float) -> "Dataset":
        out = C.c_void_p()
        self._check(self._L.seeml_hip_dataset_split_validation(self._h, C.c_double(fraction), C.byref(out)))
        return Dataset(out)


def splitmix64(state: int) -> tuple[int, int]:
    """(new state, output) of one splitmix64 step, from the native code."""
    s = C.c_uint64(state)
    out = _lib.lib().seeml_hip_splitmix64(C.byref(s))
    return s.value, out
