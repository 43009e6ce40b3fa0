"""Batch feeder: the native Dataset (csrc/feeder.cc) against the oracle
restatement (oracle/feeder_oracle.py), bit for bit, and both against the
reference's own dataset tests (test/runtime/feeder/dataset_test.cc) and the
published splitmix64 outputs. Host only: no GPU is touched."""
import os
import struct
import tempfile

import numpy as np
import pytest

import feeder_oracle as fo
from seeml_amd import feeder as nf


def marker(n=64, dim=4):
    """dataset_test.cc:220-238 MarkerDataset: feature 0 = sample index, label = index % 2."""
    x = np.repeat(np.arange(n, dtype=np.float32), dim)
    lab = (np.arange(n) % 2).astype(np.int32).tobytes()
    return x, lab, n, dim


def both_marker(n=64, dim=4):
    x, lab, n, dim = marker(n, dim)
    return (nf.Dataset.from_memory(x, lab, n, dim, 1), fo.Dataset.from_memory(x, lab, n, dim, 1, 0))


def test_splitmix64_published_outputs():
    want = [0xE220A8397B1DCDAF, 0x6E789E6AA1B965F4, 0x06C45D188009454F, 0xF88BB8A8724C81EC]
    s_o = s_n = 0
    for w in want:
        s_o, o = fo.splitmix64(s_o)
        s_n, n = nf.splitmix64(s_n)
        assert o == w and n == w and s_o == s_n


@pytest.mark.parametrize("n", [1, 2, 3, 5, 8])
def test_every_epoch_is_a_permutation(n):
    d = fo.Dataset.from_memory(np.arange(n, dtype=np.float32), b"", n, 1, 0, 0)
    d.enable_shuffle(3)
    for _ in range(6):
        assert sorted(d.order) == list(range(n))
        d.reshuffle()


def test_fisher_yates_matches_transcription():
    # Brute force on tiny n: the permutation equals an independent swap loop
    # over the same splitmix64 draws.
    for n in range(1, 7):
        for seed in range(5):
            d = fo.Dataset.from_memory(np.arange(n, dtype=np.float32), b"", n, 1, 0, 0)
            d.enable_shuffle(seed)
            st, out = fo.splitmix64(seed)
            st = out | 1
            perm = list(range(n))
            for i in range(n - 1, 0, -1):
                st, r = fo.splitmix64(st)
                j = r % (i + 1)
                perm[i], perm[j] = perm[j], perm[i]
            assert d.order == perm


def test_reference_wraparound_and_null_labels():
    # dataset_test.cc:92-120
    for make in (lambda *a: nf.Dataset.from_memory(*a[:5]), fo.Dataset.from_memory):
        d = make([0, 1, 10, 11, 20, 21], np.array([0, 1, 2], np.int32).tobytes(), 3, 2, 1, 0)
        x, lab = d.fill_batch(2)
        x = np.frombuffer(x, np.float32) if isinstance(x, bytes) else x
        assert x[0] == 0.0 and x[2] == 10.0 and list(np.frombuffer(lab, np.int32)) == [0, 1]
        x, lab = d.fill_batch(2)
        x = np.frombuffer(x, np.float32) if isinstance(x, bytes) else x
        assert x[0] == 20.0 and x[2] == 0.0 and list(np.frombuffer(lab, np.int32)) == [2, 0]
    d = nf.Dataset.from_memory([1, 2, 3], b"", 3, 1, 0)
    x, lab = d.fill_batch(2, labels=False)
    assert list(x) == [1.0, 2.0] and lab == b""


def test_reference_token_shift_and_bounds():
    # dataset_test.cc:275-291
    d = nf.Dataset.from_tokens(list(range(8)), 2, 3)
    assert d.input_kind == 1 and d.label_kind == 1
    x, lab = d.fill_batch(6)
    assert list(x) == [0, 1, 2, 4, 5, 6]
    assert list(np.frombuffer(lab, np.int32)) == [1, 2, 3, 5, 6, 7]
    d.validate_class_labels(8)
    with pytest.raises(RuntimeError, match="outside"):
        d.validate_class_labels(7)


def test_reference_shuffle_determinism_and_coverage():
    # dataset_test.cc:240-273
    a, _ = both_marker()
    b, _ = both_marker()
    a.enable_shuffle(9)
    b.enable_shuffle(9)
    seen = np.zeros(64, int)
    permuted = False
    for batch in range(8):
        xa, la = a.fill_batch(8)
        xb, lb = b.fill_batch(8)
        assert np.array_equal(xa, xb) and la == lb
        ids = xa.reshape(8, 4)[:, 0].astype(int)
        labs = np.frombuffer(la, np.int32)
        for i, idx in enumerate(ids):
            seen[idx] += 1
            permuted |= idx != batch * 8 + i
            assert labs[i] == idx % 2
    assert np.all(seen == 1) and permuted
    xa, _ = a.fill_batch(8)
    xb, _ = b.fill_batch(8)
    assert np.array_equal(xa, xb)


def test_reference_restore_replays_across_epochs():
    # dataset_test.cc:317-346
    d, _ = both_marker()
    d.enable_shuffle(17)
    d.fill_batch(8)
    snap = d.serving_pos()
    want = [d.fill_batch(8)[0] for _ in range(24)]
    d.restore_serving_pos(*snap)
    for w in want:
        assert np.array_equal(d.fill_batch(8)[0], w)


def test_reference_split_tail_and_rejections():
    # dataset_test.cc:348-373
    d, _ = both_marker()
    v = d.split_validation(0.25)
    assert d.num_samples == 48 and v.num_samples == 16
    x, _ = v.fill_batch(1)
    assert int(x[0]) == 48
    d, _ = both_marker()
    for f in (0.0, 1.0):
        with pytest.raises(RuntimeError, match="fraction"):
            d.split_validation(f)
    d.enable_shuffle(1)
    with pytest.raises(RuntimeError, match="before enabling shuffle"):
        d.split_validation(0.25)


def test_token_records_roundtrip_split_shuffle():
    # dataset_test.cc:293-315 with a successor-property corpus: each record
    # is consecutive ids, so any cross-record mixing shows immediately.
    seq, n = 4, 8
    toks = np.concatenate([np.arange(r * 16, r * 16 + seq + 1) for r in range(n)]).astype(np.int32)
    d = nf.Dataset.from_tokens(toks, n, seq)
    with tempfile.TemporaryDirectory() as tmp:
        path = os.path.join(tmp, "t.sds")
        d.save(path)
        raw = open(path, "rb").read()
        assert raw == fo.Dataset.from_tokens(toks, n, seq).to_sds()
        loaded = nf.Dataset.load(path)
    assert loaded.input_kind == 1 and loaded.num_samples == 8 and loaded.input_dim == 4
    val = loaded.split_validation(0.25)
    assert val.num_samples == 2 and loaded.num_samples == 6
    loaded.enable_shuffle(5)
    x, lab = loaded.fill_batch(24)
    lab = np.frombuffer(lab, np.int32)
    for r in range(6):
        for i in range(3):
            assert lab[r * 4 + i] == x[r * 4 + i + 1]


@pytest.mark.parametrize("seed", [0, 1, 9, 12345, 2**63 + 7])
def test_native_matches_oracle_feature_rows(seed):
    rng = np.random.default_rng(seed % 1000)
    n, dim = 37, 5
    x = rng.standard_normal(n * dim).astype(np.float32)
    lab = rng.integers(0, 10, n).astype(np.int32).tobytes()
    a = nf.Dataset.from_memory(x, lab, n, dim, 1)
    b = fo.Dataset.from_memory(x, lab, n, dim, 1, 0)
    for d in (a, b):
        d.enable_shuffle(seed)
    for step in range(40):  # > 3 epochs at batch 7 (epochs wrap mid-batch)
        xa, la = a.fill_batch(7)
        xb, lb = b.fill_batch(7)
        assert xa.tobytes() == xb and la == lb, step
        assert a.serving_pos() == b.serving_pos()
    # resume replay (the checkpoint path): skip then serve
    for d in (a, b):
        d.skip_served(7 * 29)
    assert a.serving_pos() == b.serving_pos()
    assert a.fill_batch(7)[0].tobytes() == b.fill_batch(7)[0]


def test_native_matches_oracle_tokens_sequential_and_shuffled():
    rng = np.random.default_rng(4)
    n, seq = 11, 6
    toks = rng.integers(0, 50, n * (seq + 1)).astype(np.int32)
    for shuffle in (None, 77):
        a = nf.Dataset.from_tokens(toks, n, seq)
        b = fo.Dataset.from_tokens(toks, n, seq)
        if shuffle is not None:
            a.enable_shuffle(shuffle)
            b.enable_shuffle(shuffle)
        for step in range(25):
            xa, la = a.fill_batch(3 * seq)
            xb, lb = b.fill_batch(3 * seq)
            assert xa.tobytes() == xb and la == lb, (shuffle, step)
    with pytest.raises(RuntimeError, match="whole number of token records"):
        a.skip_served(seq + 1)


def test_dense_labels_file_roundtrip_bytes():
    rng = np.random.default_rng(2)
    n, dim, ldim = 9, 3, 2
    x = rng.standard_normal(n * dim).astype(np.float32)
    lab = rng.standard_normal(n * ldim).astype(np.float32).tobytes()
    d = nf.Dataset.from_memory(x, lab, n, dim, 2, ldim)
    assert d.label_bytes_per_sample() == 8
    with tempfile.TemporaryDirectory() as tmp:
        path = os.path.join(tmp, "d.sds")
        d.save(path)
        assert open(path, "rb").read() == fo.Dataset.from_memory(x, lab, n, dim, 2, ldim).to_sds()
        e = nf.Dataset.load(path)
    assert e.fill_batch(n)[1] == lab


def sds_header(magic, version, n, dim, label_kind, label_dim, input_kind=0):
    return struct.pack("<IIQQIIQ", magic, version, n, dim, label_kind, input_kind, label_dim)


@pytest.mark.parametrize("blob,msg", [
    (b"XXXX", "bad magic"),
    (sds_header(fo.SDS_MAGIC, 3, 1, 1, 0, 0), "unsupported version"),
    (struct.pack("<II", fo.SDS_MAGIC, 1) + b"\0" * 8, "truncated header"),
    (sds_header(fo.SDS_MAGIC, 1, 0, 1, 0, 0), "empty dataset"),
    (sds_header(fo.SDS_MAGIC, 1, 1, 1, 3, 0), "unknown label kind"),
    (sds_header(fo.SDS_MAGIC, 1, 1, 1, 2, 0), "label dim out of range"),
    (sds_header(fo.SDS_MAGIC, 1, 4, 2, 1, 0) + b"\0" * 8, "exceeds file size"),
    (sds_header(fo.SDS_MAGIC, 1, 1, 1, 0, 0, input_kind=1), "unknown input kind"),
    (sds_header(fo.SDS_MAGIC, 2, 1, 2, 1, 0, input_kind=1) + struct.pack("<iii", 1, -2, 3),
     "negative token id"),
])
def test_load_rejects_malformed_files(blob, msg):
    # dataset_test.cc:182-217
    with tempfile.TemporaryDirectory() as tmp:
        path = os.path.join(tmp, "bad.sds")
        open(path, "wb").write(blob)
        with pytest.raises(RuntimeError, match=msg):
            nf.Dataset.load(path)
    with pytest.raises(RuntimeError, match="cannot open"):
        nf.Dataset.load("/nonexistent/x.sds")


def test_constructor_rejections():
    with pytest.raises(RuntimeError, match="token buffer size mismatch"):
        nf.Dataset.from_tokens([1, 2, 3], 1, 3)
    with pytest.raises(RuntimeError, match="negative token id at position 1"):
        nf.Dataset.from_tokens([1, -1, 3, 4], 1, 3)
    with pytest.raises(RuntimeError, match="label buffer size mismatch"):
        nf.Dataset.from_memory([1, 2], b"\0" * 3, 2, 1, 1)
    with pytest.raises(RuntimeError, match="class label 5 at sample 1 outside \\[0, 3\\)"):
        nf.Dataset.from_memory([1, 2], np.array([0, 5], np.int32).tobytes(), 2, 1, 1).validate_class_labels(3)


def test_argmax_oracle_semantics():
    # The sequential strict-'>' scan: ties -> lowest index, NaN never wins,
    # NaN in column 0 pins index 0, -0 == +0, negative labels never count.
    nan = np.nan
    probs = np.array([[0.1, 0.5, 0.5], [nan, 0.9, 0.2], [0.2, nan, 0.3], [-0.0, 0.0, -1.0],
                      [0.3, 0.2, 0.1]], np.float32)
    assert fo.argmax_hits(probs, np.array([1, 0, 2, 0, -1])) == 4
    assert fo.argmax_hits(probs, np.array([2, 1, 1, 1, 0])) == 1
