"""seeml_amd — MI355X (gfx950) backend for SeeML's compiled LoRA update step.

The product is the C-ABI library (include/seeml_hip.h, built from csrc/ into
lib/libseeml_hip.so). This package is its host-side surface:
  _lib       ctypes binding generated from the header
  engine     DeviceUpdateEngine, the UpdateEngine-shaped wrapper
  feeder     Dataset, the native batch feeder's dataset
  planner    the compiler pipeline restated to produce .seeu plans
  configs    the BASELINE workloads and their synthetic batches
"""
from . import configs, feeder, planner  # noqa: F401
from ._lib import lib  # noqa: F401
from .engine import DeviceUpdateEngine, PROGRAM_EVAL, PROGRAM_MERGE, PROGRAM_TRAIN  # noqa: F401
