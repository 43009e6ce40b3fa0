"""The SEKP checkpoint container (runtime/custodian/checkpoint.{h,cc}),
host only: the byte layout, the payload hash against the reference's own
ContentHash64 (oracle/_ref), a durable write that leaves no temporary file,
and every rejection the reference makes, with dst untouched."""
import ctypes as C
import os
import struct
import tempfile

import numpy as np
import pytest

from seeml_amd import _lib

MAGIC = 0x504B4553


def write(path, plan_hash, step, payload):
    err = C.create_string_buffer(512)
    buf = (C.c_uint8 * max(len(payload), 1)).from_buffer_copy(payload or b"\0")
    rc = _lib.lib().seeml_hip_checkpoint_write(path.encode(), plan_hash, step, buf, len(payload),
                                               err, 512)
    return rc, err.value.decode()


def read(path, plan_hash, size):
    err = C.create_string_buffer(512)
    dst = (C.c_uint8 * max(size, 1))(*([0xAB] * max(size, 1)))
    step = C.c_uint64(0)
    rc = _lib.lib().seeml_hip_checkpoint_read(path.encode(), plan_hash, size, dst, C.byref(step),
                                              err, 512)
    return rc, err.value.decode(), bytes(dst)[:size], step.value


def test_layout_round_trip_and_reference_hash(ref):
    payload = np.random.default_rng(3).standard_normal(70001).astype(np.float32).tobytes()
    with tempfile.TemporaryDirectory() as d:
        path = os.path.join(d, "ck.sekp")
        assert write(path, 0x1234ABCD5678, 42, payload) == (0, "")
        assert sorted(os.listdir(d)) == ["ck.sekp"]  # the temporary file was renamed
        raw = open(path, "rb").read()
        magic, version, ph, step, size, phash = struct.unpack_from("<IIQQQQ", raw, 0)
        assert (magic, version, ph, step, size) == (MAGIC, 3, 0x1234ABCD5678, 42, len(payload))
        assert phash == ref.content_hash64(payload, len(payload))
        assert raw[40:] == payload and len(raw) == 40 + len(payload)
        rc, msg, got, st = read(path, 0x1234ABCD5678, len(payload))
        assert (rc, msg, got, st) == (0, "", payload, 42)


def test_rejections_leave_dst_untouched():
    payload = bytes(range(256)) * 8
    n = len(payload)
    with tempfile.TemporaryDirectory() as d:
        good = os.path.join(d, "good")
        assert write(good, 7, 3, payload)[0] == 0
        raw = open(good, "rb").read()

        def variant(name, blob):
            p = os.path.join(d, name)
            open(p, "wb").write(blob)
            return p

        bad_magic = variant("magic", b"XXXX" + raw[4:])
        v2 = variant("v2", raw[:4] + struct.pack("<I", 2) + raw[8:])
        short_header = variant("short", raw[:20])
        truncated = variant("trunc", raw[:-1])
        corrupt = variant("corrupt", raw[:100] + bytes([raw[100] ^ 1]) + raw[101:])
        cases = [
            (os.path.join(d, "missing"), 7, n, "Checkpoint: no checkpoint at"),
            (bad_magic, 7, n, "Checkpoint: not a v3 checkpoint"),
            (v2, 7, n, "Checkpoint: not a v3 checkpoint"),
            (short_header, 7, n, "Checkpoint: not a v3 checkpoint"),
            (good, 8, n, "Checkpoint: checkpoint belongs to a different plan"),
            (good, 7, n - 4, "Checkpoint: checkpoint incompatible with plan"),
            (truncated, 7, n, "Checkpoint: truncated checkpoint"),
            (corrupt, 7, n, "Checkpoint: checkpoint payload is corrupt"),
        ]
        for path, plan_hash, size, want in cases:
            rc, msg, got, step = read(path, plan_hash, size)
            assert rc == 1 and msg.startswith(want), (path, msg)
            assert got == bytes([0xAB]) * size and step == 0, path
        rc, msg = write(os.path.join(d, "no_such_dir", "x"), 1, 1, payload)
        assert rc == 1 and msg.startswith("Checkpoint: cannot write"), msg
