"""Feeder oracle — TEST INFRASTRUCTURE ONLY.

A plain-Python restatement of the reference's batch feeder dataset
(runtime/feeder/dataset.cc) used by tests/ to check the product's native
feeder (see-ml_amd/csrc/feeder.cc) bit for bit. Nothing in the product path
imports this module.

Pins (tests/test_feeder.py):
  * splitmix64 against the published seed-0 outputs of the algorithm
    (e220a8397b1dcdaf, 6e789e6aa1b965f4, 06c45d188009454f, f88bb8a8724c81ec);
  * Fisher-Yates: every epoch is a permutation, and the swap sequence is
    checked by brute force on tiny n against a direct transcription;
  * the reference's own dataset tests' known answers
    (test/runtime/feeder/dataset_test.cc: wraparound order, shifted token
    labels, shuffle determinism and epoch coverage, deep restore replay,
    split tails, rejection messages).
"""
from __future__ import annotations

import struct

import numpy as np

M64 = (1 << 64) - 1
SDS_MAGIC = 0x31534453


def splitmix64(state: int) -> tuple[int, int]:
    """One splitmix64 step (dataset.cc:344-352): (new_state, output)."""
    state = (state + 0x9E3779B97F4A7C15) & M64
    z = state
    z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & M64
    z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & M64
    return state, z ^ (z >> 31)


class FeedError(ValueError):
    pass


class Dataset:
    """Dataset (dataset.h:39-177). Inputs are np.float32 [n, dim] (feature
    rows) or the token stream np.int32 [n*(seq+1)]; labels are raw bytes."""

    def __init__(self):
        self.inputs = None
        self.labels = b""
        self.tokens = None
        self.num_samples = 0
        self.input_dim = 0
        self.label_kind = 0
        self.input_kind = 0
        self.label_dim = 0
        self.cursor = 0
        self.order: list[int] = []
        self.state = 0
        self.origin = 0
        self.epoch = 0

    # -- construction (dataset.cc:34-84) ------------------------------------
    @staticmethod
    def from_tokens(tokens, num_records: int, seq: int) -> "Dataset":
        tokens = np.asarray(tokens, np.int32)
        if num_records == 0:
            raise FeedError("Dataset: zero samples")
        if seq == 0:
            raise FeedError("Dataset: zero input dim")
        if tokens.size != num_records * (seq + 1):
            raise FeedError("Dataset: token buffer size mismatch")
        neg = np.flatnonzero(tokens < 0)
        if neg.size:
            raise FeedError(f"Dataset: negative token id at position {neg[0]}")
        d = Dataset()
        d.input_kind, d.label_kind = 1, 1
        d.num_samples, d.input_dim = num_records, seq
        d.tokens = tokens.copy()
        return d

    @staticmethod
    def from_memory(inputs, labels: bytes, num_samples: int, input_dim: int,
                    label_kind: int, label_dim: int) -> "Dataset":
        d = Dataset()
        d.num_samples, d.input_dim = num_samples, input_dim
        d.label_kind, d.label_dim = label_kind, label_dim
        if num_samples == 0:
            raise FeedError("Dataset: zero samples")
        if input_dim == 0:
            raise FeedError("Dataset: zero input dim")
        if label_kind > 2:
            raise FeedError("Dataset: unknown label kind")
        if label_kind == 2 and label_dim == 0:
            raise FeedError("Dataset: label dim out of range")
        inputs = np.asarray(inputs, np.float32).reshape(-1)
        if inputs.size != num_samples * input_dim:
            raise FeedError("Dataset: input buffer size mismatch")
        if len(labels) != num_samples * d.label_bytes_per_sample():
            raise FeedError("Dataset: label buffer size mismatch")
        d.inputs = inputs.reshape(num_samples, input_dim).copy()
        d.labels = bytes(labels)
        return d

    def label_bytes_per_sample(self) -> int:
        """dataset.cc:23-33."""
        if self.input_kind == 1:
            return self.input_dim * 4
        return {1: 4, 2: self.label_dim * 4}.get(self.label_kind, 0)

    def validate_class_labels(self, num_classes: int) -> None:
        """dataset.cc:199-228."""
        if self.label_kind != 1 or num_classes == 0:
            return
        if self.input_kind == 1:
            for i, t in enumerate(self.tokens.tolist()):
                if t < 0 or t >= num_classes:
                    raise FeedError(f"Dataset: token id {t} at position {i} outside [0, {num_classes})")
            return
        labs = np.frombuffer(self.labels, np.int32)
        for i, v in enumerate(labs.tolist()):
            if v < 0 or v >= num_classes:
                raise FeedError(f"Dataset: class label {v} at sample {i} outside [0, {num_classes})")

    # -- serving (dataset.cc:288-342) -----------------------------------------
    def _advance(self) -> None:
        self.cursor += 1
        if self.cursor == self.num_samples:
            self.cursor = 0
            if self.order:
                self.reshuffle()
                self.epoch += 1

    def fill_batch(self, batch: int):
        """Returns (inputs bytes, labels bytes) of the next `batch` rows."""
        lb = self.label_bytes_per_sample()
        if self.input_kind == 1:
            S = self.input_dim
            ins, labs = [], []
            for _ in range(batch // S):
                i = self.order[self.cursor] if self.order else self.cursor
                rec = self.tokens[i * (S + 1):(i + 1) * (S + 1)]
                ins.append(rec[:S].tobytes())
                labs.append(rec[1:].tobytes())
                self._advance()
            return b"".join(ins), b"".join(labs)
        ins, labs = [], []
        for _ in range(batch):
            i = self.order[self.cursor] if self.order else self.cursor
            ins.append(self.inputs[i].tobytes())
            labs.append(self.labels[i * lb:(i + 1) * lb])
            if self.order:
                self._advance()
            else:
                self.cursor += 1
                if self.cursor == self.num_samples:
                    self.cursor = 0
        return b"".join(ins), b"".join(labs)

    # -- shuffling (dataset.cc:356-417) ----------------------------------------
    def enable_shuffle(self, seed: int) -> None:
        self.state, out = splitmix64(seed & M64)
        self.state = out | 1
        self.origin = self.state
        self.epoch = 0
        self.order = list(range(self.num_samples))
        self.reshuffle()
        self.cursor = 0

    def reshuffle(self) -> None:
        order = list(range(self.num_samples))
        for i in range(self.num_samples - 1, 0, -1):
            self.state, r = splitmix64(self.state)
            j = r % (i + 1)
            order[i], order[j] = order[j], order[i]
        self.order = order

    def serving_pos(self) -> tuple[int, int]:
        return self.cursor, self.epoch

    def restore_serving_pos(self, cursor: int, epoch: int) -> None:
        self.cursor = cursor
        if not self.order or self.epoch == epoch:
            return
        self.state = self.origin
        self.epoch = 0
        self.reshuffle()
        while self.epoch < epoch:
            self.reshuffle()
            self.epoch += 1

    def skip_served(self, rows: int) -> None:
        records = rows
        if self.input_kind == 1:
            if rows % self.input_dim:
                raise FeedError("Dataset: served rows are not a whole number of token records")
            records = rows // self.input_dim
        self.restore_serving_pos(records % self.num_samples, records // self.num_samples)

    def split_validation(self, fraction: float) -> "Dataset":
        """dataset.cc:419-462: the tail moves, at least one sample each side."""
        if not (fraction > 0.0) or fraction >= 1.0:
            raise FeedError("Dataset: validation fraction must be in (0, 1)")
        if self.num_samples < 2:
            raise FeedError("Dataset: too few samples to split")
        if self.order:
            raise FeedError("Dataset: split before enabling shuffle")
        val_n = int(float(self.num_samples) * fraction)
        val_n = min(max(val_n, 1), self.num_samples - 1)
        train_n = self.num_samples - val_n
        v = Dataset()
        v.num_samples, v.input_dim = val_n, self.input_dim
        v.label_kind, v.label_dim, v.input_kind = self.label_kind, self.label_dim, self.input_kind
        if self.input_kind == 1:
            rec = self.input_dim + 1
            v.tokens = self.tokens[train_n * rec:].copy()
            self.tokens = self.tokens[:train_n * rec].copy()
        else:
            lb = self.label_bytes_per_sample()
            v.inputs = self.inputs[train_n:].copy()
            v.labels = self.labels[train_n * lb:]
            self.inputs = self.inputs[:train_n].copy()
            self.labels = self.labels[:train_n * lb]
        self.num_samples = train_n
        self.cursor = 0
        return v

    # -- .sds bytes (dataset.cc:230-286) -----------------------------------------
    def to_sds(self) -> bytes:
        version = 2 if self.input_kind == 1 else 1
        head = struct.pack("<IIQQIIQ", SDS_MAGIC, version, self.num_samples, self.input_dim,
                           self.label_kind, self.input_kind, self.label_dim)
        if self.input_kind == 1:
            return head + self.tokens.tobytes()
        lb = self.label_bytes_per_sample()
        body = b"".join(self.inputs[i].tobytes() + self.labels[i * lb:(i + 1) * lb]
                        for i in range(self.num_samples))
        return head + body


def argmax_hits(probs: np.ndarray, labels: np.ndarray) -> int:
    """EvaluateMetrics' accuracy count (update_engine.cc:619-633): the
    sequential strict-'>' scan from column 0 per row, label match counted
    when the label is non-negative."""
    hits = 0
    for r in range(probs.shape[0]):
        row = probs[r]
        best = 0
        for c in range(1, row.shape[0]):
            if row[c] > row[best]:
                best = c
        if labels[r] >= 0 and int(labels[r]) == best:
            hits += 1
    return hits
