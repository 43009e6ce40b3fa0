"""Host-side mirror of the reference's UpdateEngine surface over the C-ABI.

UpdateEngine (runtime/engine/update_engine.h:119-242) -> DeviceUpdateEngine:
  LoadFromMemory            -> DeviceUpdateEngine(plan_bytes)       (seeml_hip_open)
  ExecuteTrainOnce / Train  -> train_step / train                   (seeml_hip_train_step)
  LossValue                 -> loss()
  Evaluate                  -> evaluate(batches)  (eval program + double mean)
  Train(Dataset&, ...)      -> train_dataset(dataset, steps, validation)
  EvaluateMetrics(Dataset&) -> evaluate_metrics(dataset)  (loss + argmax accuracy)
  RunMerge                  -> run_merge()
  arena probes              -> read / write (test/support/probes.cc:25-60)
Errors surface as RuntimeError carrying the "<unit>: <message>" text.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from . import _lib

PROGRAM_TRAIN, PROGRAM_MERGE, PROGRAM_EVAL = 0, 1, 2


class _EvalMetrics(C.Structure):
    _fields_ = [("loss", C.c_float), ("has_accuracy", C.c_int32), ("accuracy", C.c_float)]


_SHOULD_STOP = C.CFUNCTYPE(C.c_int, C.c_void_p)


class _TrainOptions(C.Structure):
    _fields_ = [("checkpoint_path", C.c_char_p), ("checkpoint_every", C.c_uint64),
                ("resume", C.c_int32), ("should_stop", C.c_void_p),
                ("should_stop_ctx", C.c_void_p)]


class _TrainReport(C.Structure):
    _fields_ = [("steps", C.c_uint64), ("initial_avg_loss", C.c_float),
                ("final_avg_loss", C.c_float), ("has_validation", C.c_int32),
                ("val_initial_loss", C.c_float), ("val_final_loss", C.c_float),
                ("has_val_accuracy", C.c_int32), ("val_initial_accuracy", C.c_float),
                ("val_final_accuracy", C.c_float), ("improved", C.c_int32),
                ("stopped_early", C.c_int32)]


def _buf(a):
    """(pointer, nbytes, on_device) for a numpy array or a torch tensor."""
    if a is None:
        return None, 0, 0
    if isinstance(a, np.ndarray):
        a = np.ascontiguousarray(a)
        return a.ctypes.data, a.nbytes, 0
    # torch tensor (device-resident staging)
    return a.data_ptr(), a.numel() * a.element_size(), 1 if a.is_cuda else 0


class DeviceUpdateEngine:
    def __init__(self, plan: bytes, device: int = 0, use_graph: bool = True):
        self._L = _lib.lib()
        err = C.create_string_buffer(1024)
        h = C.c_void_p()
        view = np.frombuffer(plan, np.uint8)  # no copy; the library reads only
        rc = self._L.seeml_hip_open(view.ctypes.data, len(plan), device, C.byref(h), err, len(err))
        del view
        if rc != 0:
            raise RuntimeError(err.value.decode())
        self._h = h
        if not use_graph:
            self._L.seeml_hip_set_graph_mode(self._h, 0)

    def close(self):
        if getattr(self, "_h", None):
            self._L.seeml_hip_close(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def _check(self, rc, what):
        if rc != 0:
            raise RuntimeError(f"{what}: {self._L.seeml_hip_last_error(self._h).decode()}")

    # -- lifecycle ----------------------------------------------------------
    def build(self, program: int = PROGRAM_TRAIN):
        self._check(self._L.seeml_hip_build(self._h, program), "build")

    def set_step(self, step: int):
        self._check(self._L.seeml_hip_set_step(self._h, step), "set_step")

    @property
    def step(self) -> int:
        return self._L.seeml_hip_get_step(self._h)

    def stage(self, inputs, labels=None):
        ip, ib, idev = _buf(inputs)
        lp, lb, ldev = _buf(labels)
        self._check(self._L.seeml_hip_stage(self._h, ip, ib, lp, lb, idev or ldev), "stage")

    def run(self, program: int = PROGRAM_TRAIN):
        self._check(self._L.seeml_hip_run(self._h, program), "run")

    def run_range(self, program: int, begin: int, end: int):
        """Instructions [begin, end) of `program`, each once, eagerly."""
        self._check(self._L.seeml_hip_run_range(self._h, program, begin, end), "run_range")

    def sync(self):
        self._check(self._L.seeml_hip_sync(self._h), "sync")

    def loss(self) -> float:
        out = C.c_float()
        self._check(self._L.seeml_hip_loss(self._h, C.byref(out)), "loss")
        return out.value

    def train_step(self, inputs, labels=None) -> float:
        ip, ib, idev = _buf(inputs)
        lp, lb, ldev = _buf(labels)
        out = C.c_float()
        self._check(self._L.seeml_hip_train_step(self._h, ip, ib, lp, lb, idev or ldev,
                                                 C.byref(out)), "train_step")
        return out.value

    def train(self, batches) -> list:
        return [self.train_step(x, y) for x, y in batches]

    def evaluate(self, batches) -> float:
        """Evaluate's loss: eval program per batch, mean of f32 losses in
        double (update_engine.cc:603-643)."""
        total, n = 0.0, 0
        for x, y in batches:
            self.stage(x, y)
            self.run(PROGRAM_EVAL)
            total += self.loss()
            n += 1
        return float(np.float32(total / max(n, 1)))

    def evaluate_metrics(self, dataset) -> dict:
        """EvaluateMetrics (update_engine.cc:557-650) over a feeder Dataset."""
        m = _EvalMetrics()
        self._check(self._L.seeml_hip_evaluate_metrics(self._h, dataset._h, C.byref(m)),
                    "evaluate_metrics")
        return dict(loss=m.loss, has_accuracy=bool(m.has_accuracy), accuracy=m.accuracy)

    def train_dataset(self, dataset, steps: int = 0, validation=None, checkpoint_path=None,
                      checkpoint_every: int = 0, resume: bool = False,
                      should_stop=None) -> dict:
        """TrainImpl (update_engine.cc:664-787) with the native feeder and
        TrainOptions (checkpointing, resume, should_stop polled once per
        step); the report's loss_curve holds every step's loss."""
        r = _TrainReport()
        cap = steps if steps else 0
        curve = np.zeros(max(cap, 1), np.float32)
        stop_cb = _SHOULD_STOP(lambda _ctx: 1 if should_stop() else 0) if should_stop else None
        opt = _TrainOptions(checkpoint_path.encode() if checkpoint_path else None,
                            checkpoint_every, 1 if resume else 0,
                            C.cast(stop_cb, C.c_void_p) if stop_cb else None, None)
        self._check(self._L.seeml_hip_train_ex(self._h, dataset._h, steps,
                                               validation._h if validation is not None else None,
                                               curve.ctypes.data, cap, C.byref(opt), C.byref(r)),
                    "train")
        out = {f: getattr(r, f) for f, _ in _TrainReport._fields_}
        for k in ("has_validation", "has_val_accuracy", "improved", "stopped_early"):
            out[k] = bool(out[k])
        out["loss_curve"] = curve[:min(cap, r.steps)]
        return out

    def save_checkpoint(self, path: str):
        self._check(self._L.seeml_hip_save_checkpoint(self._h, path.encode()), "save_checkpoint")

    def load_checkpoint(self, path: str):
        self._check(self._L.seeml_hip_load_checkpoint(self._h, path.encode()), "load_checkpoint")

    def run_merge(self):
        self._check(self._L.seeml_hip_run_merge(self._h), "run_merge")

    def autotune(self, budget: int = 16):
        self._check(self._L.seeml_hip_autotune(self._h, budget), "autotune")

    def gemm_choice(self, program: int, index: int) -> str:
        buf = C.create_string_buffer(128)
        self._check(self._L.seeml_hip_gemm_choice(self._h, program, index, buf, len(buf)),
                    "gemm_choice")
        return buf.value.decode()

    def launch_work(self, program: int, index: int):
        """(flops, bytes) of the fused launch instruction `index`'s profile
        row carries, or None where the instruction's own work applies."""
        f, b = C.c_double(), C.c_double()
        self._check(self._L.seeml_hip_launch_work(self._h, program, index, C.byref(f), C.byref(b)),
                    "launch_work")
        return None if f.value < 0 else (f.value, b.value)

    def program_length(self, program: int = PROGRAM_TRAIN) -> int:
        return self._L.seeml_hip_program_length(self._h, program)

    def profile(self, program: int = PROGRAM_TRAIN, reps: int = 3) -> np.ndarray:
        """Per-instruction mean ms (HIP events on the engine stream, eager)."""
        n = self.program_length(program)
        out = np.zeros(max(n, 1), np.float32)
        self._check(self._L.seeml_hip_profile_program(self._h, program, reps, out.ctypes.data, n),
                    "profile")
        return out[:n]

    def mark_timed(self, program: int, indices) -> None:
        """Event-record nodes around these instructions in the program's
        graph: ordinary replays then time them (marked_times)."""
        idx = np.ascontiguousarray(sorted(set(int(i) for i in indices)), np.uint64)
        self._check(self._L.seeml_hip_mark_timed(self._h, program, idx.ctypes.data, idx.size),
                    "mark_timed")
        self._marked = idx.size

    def marked_times(self, program: int = PROGRAM_TRAIN) -> np.ndarray:
        """ms of each marked launch in the latest completed replay."""
        out = np.zeros(max(getattr(self, "_marked", 0), 1), np.float32)
        self._check(self._L.seeml_hip_marked_times(self._h, program, out.ctypes.data, out.size),
                    "marked_times")
        return out[:getattr(self, "_marked", 0)]

    def time_instruction(self, program: int, index: int, reps: int = 10) -> float:
        out = C.c_float()
        self._check(self._L.seeml_hip_time_instruction(self._h, program, index, reps, C.byref(out)),
                    "time_instruction")
        return out.value

    # -- probes ---------------------------------------------------------------
    def read(self, ref: int, count: int, dtype=np.float32) -> np.ndarray:
        out = np.empty(count, dtype)
        self._check(self._L.seeml_hip_read(self._h, ref, out.ctypes.data, out.nbytes), "read")
        return out

    def write(self, ref: int, data: np.ndarray):
        data = np.ascontiguousarray(data)
        self._check(self._L.seeml_hip_write(self._h, ref, data.ctypes.data, data.nbytes), "write")

    @property
    def stream(self) -> int:
        return self._L.seeml_hip_stream(self._h) or 0

    @property
    def arena_ptr(self) -> int:
        return self._L.seeml_hip_arena_device_ptr(self._h) or 0
