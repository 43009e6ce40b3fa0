"""ctypes bindings for the CPU oracles — TEST INFRASTRUCTURE ONLY.

Two libraries share one signature table:
  * ``liboracle.so`` (prefix ``orc_``): this build's C restatement of the
    reference executor (seeml_oracle.c);
  * ``_ref/libseeml_ref.so`` (prefix ``ref_``): the reference's own executor
    sources compiled in place (oracle/Makefile) — present where
    /root/reference was available at build time.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
import this module; the product path never does.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_SO = os.path.join(HERE, "liboracle.so")
REF_SO = os.path.join(HERE, "_ref", "libseeml_ref.so")

_P = C.c_void_p
_Z = C.c_size_t
_F = C.c_float
_I = C.c_int
_U64 = C.c_uint64

# name -> argtypes (restype void unless listed in _RESTYPES)
SIGNATURES = {
    "gemm_nn": [_P, _P, _P, _Z, _Z, _Z, _P, _I],
    "gemm_nt": [_P, _P, _P, _Z, _Z, _Z],
    "gemm_tn": [_P, _P, _P, _Z, _Z, _Z],
    "gemm_acc_nn": [_P, _P, _P, _Z, _Z, _Z, _F],
    "gemm_nn_q8": [_P, _P, _P, _Z, _Z, _Z, _F, _I],
    "gemm_nt_q8": [_P, _P, _P, _Z, _Z, _Z, _F],
    "add_ew": [_P, _P, _P, _Z],
    "mul_ew": [_P, _P, _P, _Z],
    "add_bias": [_P, _P, _P, _Z, _Z],
    "scale": [_P, _P, _F, _Z],
    "reduce_rows": [_P, _P, _Z, _Z],
    "relu_fwd": [_P, _P, _Z],
    "relu_bwd": [_P, _P, _P, _Z],
    "gelu_fwd": [_P, _P, _Z],
    "gelu_bwd": [_P, _P, _P, _Z],
    "silu_fwd": [_P, _P, _Z],
    "silu_bwd": [_P, _P, _P, _Z],
    "embed_fwd": [_P, _P, _P, _Z, _Z],
    "fill": [_P, _F, _Z],
    "copy": [_P, _P, _Z],
    "layer_norm_fwd": [_P, _P, _P, _P, _P, _P, _Z, _Z],
    "layer_norm_bwd": [_P, _P, _P, _P, _P, _P, _Z, _Z],
    "rms_norm_fwd": [_P, _P, _P, _P, _Z, _Z],
    "rms_norm_bwd": [_P, _P, _P, _P, _P, _Z, _Z],
    "rope_fwd": [_P, _P, _Z, _Z, _Z, _Z, _F],
    "rope_bwd": [_P, _P, _Z, _Z, _Z, _Z, _F],
    "attn_fwd": [_P, _P, _P, _P, _P, _Z, _Z, _Z, _Z],
    "attn_dp": [_P, _P, _P, _Z, _Z, _Z, _Z],
    "attn_dv": [_P, _P, _P, _Z, _Z, _Z, _Z],
    "softmax_rows_bwd": [_P, _P, _P, _Z, _Z],
    "attn_dq": [_P, _P, _P, _Z, _Z, _Z, _Z],
    "attn_dk": [_P, _P, _P, _Z, _Z, _Z, _Z],
    "softmax_xent_fwd": [_P, _P, _P, _P, _Z, _Z],
    "softmax_xent_bwd": [_P, _P, _P, _P, _Z, _Z],
    "mse_fwd": [_P, _P, _P, _Z],
    "mse_bwd": [_P, _P, _P, _P, _Z],
    "kl_distill_fwd": [_P, _P, _P, _P, _P, _Z, _Z, _F],
    "kl_distill_bwd": [_P, _P, _P, _P, _Z, _Z, _F],
    "clip_norm": [_P, _Z, _F],
    "sgd_step": [_P, _P, _Z, _F, _F],
    "adamw_step": [_P, _P, _P, _P, _Z, _F, _F, _F, _F, _F, _U64],
    "execute": [_P, _Z, _P, _P, _F, _F, _F, _F, _F, _U64],
}
_ORACLE_ONLY = {
    "chunk_grain": ([_Z, _Z], _Z),
    "chunk_count": ([_Z, _Z], _Z),
    "effective_lr": ([_F, C.c_uint32, _U64, _U64, _F, _U64], _F),
    "counter_randn": ([_U64, _U64, _P], None),
}
_REF_ONLY = {
    "set_threads": ([_Z], None),
    "threads": ([], _Z),
    "plan_self_hash": ([_P, _Z, _Z], _U64),
    "content_hash64": ([_P, _Z], _U64),
    "ucb1_run": ([_U64, C.c_double, _U64, _P, _P, _P, _P, _P, _P], None),
}


def _ptr(a):
    if a is None:
        return None
    if isinstance(a, np.ndarray):
        if not a.flags["C_CONTIGUOUS"]:
            raise ValueError("oracle arrays must be C-contiguous")
        return a.ctypes.data
    if isinstance(a, (bytes, bytearray)):
        return C.cast(C.c_char_p(bytes(a)), C.c_void_p).value
    return a


class KernelLib:
    """Thin wrapper: lib.gemm_nn(A, B, C, M, N, K, None, 0) with numpy arrays."""

    def __init__(self, path: str, prefix: str, extra: dict):
        self.path = path
        self.prefix = prefix
        self._lib = C.CDLL(path)
        self._fns = {}
        for name, argtypes in SIGNATURES.items():
            fn = getattr(self._lib, prefix + name)
            fn.argtypes = argtypes
            fn.restype = None
            self._fns[name] = fn
        for name, (argtypes, restype) in extra.items():
            fn = getattr(self._lib, prefix + name)
            fn.argtypes = argtypes
            fn.restype = restype
            self._fns[name] = fn

    def __getattr__(self, name):
        fns = self.__dict__.get("_fns", {})
        if name not in fns:
            raise AttributeError(name)
        fn = fns[name]

        def call(*args):
            return fn(*[_ptr(a) for a in args])

        return call


def build(ref_dir: str | None = None) -> None:
    """Build liboracle.so always, and _ref when the reference sources exist."""
    ref = ref_dir or "/root/reference"
    targets = ["oracle"]
    if os.path.isfile(os.path.join(ref, "runtime", "executor", "gemm.cc")):
        targets.append("ref")
    subprocess.check_call(["make", "-s", "-C", HERE, f"REF={ref}"] + targets)


_oracle = None
_ref = None


def oracle() -> KernelLib:
    global _oracle
    if _oracle is None:
        if not os.path.exists(ORACLE_SO):
            build()
        _oracle = KernelLib(ORACLE_SO, "orc_", _ORACLE_ONLY)
    return _oracle


def ref_available() -> bool:
    return os.path.exists(REF_SO)


def ref() -> KernelLib:
    global _ref
    if _ref is None:
        if not os.path.exists(REF_SO):
            raise FileNotFoundError(
                "oracle/_ref/libseeml_ref.so is not built (needs /root/reference)")
        _ref = KernelLib(REF_SO, "ref_", _REF_ONLY)
    return _ref
