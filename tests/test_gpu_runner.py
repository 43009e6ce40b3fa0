"""The engine-driven train / evaluate loops (UpdateEngine::Train /
EvaluateMetrics restated in csrc/engine.hip with the native feeder and the
pinned double-buffered stager) against the same loop driven from Python
with the oracle feeder through the single-step C-ABI. Same kernels, same
batches: every loss, the accuracy count and the serving position must be
identical bit for bit; the argmax kernel is checked against the sequential
strict-'>' scan."""
import ctypes as C

import numpy as np
import pytest

import feeder_oracle as fo
from seeml_amd import PROGRAM_EVAL, DeviceUpdateEngine, configs, feeder, planner

pytestmark = pytest.mark.gpu
f32 = np.float32


@pytest.fixture(scope="module")
def torch_dev():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch


def argmax_device(torch, probs, labels):
    from seeml_amd import _lib
    L = _lib.lib()
    tp = torch.from_numpy(np.ascontiguousarray(probs, f32)).cuda()
    tl = torch.from_numpy(np.ascontiguousarray(labels, np.int32)).cuda()
    out = C.c_uint64()
    rc = L.seeml_hip_argmax_correct(tp.data_ptr(), tl.data_ptr(), probs.shape[0], probs.shape[1],
                                    C.byref(out), torch.cuda.current_stream().cuda_stream)
    assert rc == 0, L.seeml_hip_kernel_error().decode()
    return out.value


def test_argmax_count_matches_sequential_scan(torch_dev):
    nan = np.nan
    probs = np.array([[0.1, 0.5, 0.5], [nan, 0.9, 0.2], [0.2, nan, 0.3], [-0.0, 0.0, -1.0],
                      [0.3, 0.2, 0.1]], f32)
    for labels in ([1, 0, 2, 0, -1], [2, 1, 1, 1, 0]):
        labels = np.array(labels, np.int32)
        assert argmax_device(torch_dev, probs, labels) == fo.argmax_hits(probs, labels)
    rng = np.random.default_rng(5)
    for rows, cols in ((1, 1), (37, 130), (513, 256), (9, 32000)):
        # coarse values make ties common; sprinkle NaNs (column 0 included)
        p = rng.integers(0, 4, (rows, cols)).astype(f32)
        p[rng.random((rows, cols)) < 0.01] = nan
        p[rng.random(rows) < 0.1, 0] = nan
        lab = rng.integers(-1, cols, rows).astype(np.int32)
        want = sum(1 for r in range(rows) if lab[r] >= 0 and lab[r] == _first_strict_argmax(p[r]))
        assert argmax_device(torch_dev, p, lab) == want, (rows, cols)


def _first_strict_argmax(row):
    best = 0
    for c in range(1, row.shape[0]):
        if row[c] > row[best]:
            best = c
    return best


def eval_probs(plan):
    ins = [i for i in plan.eval if planner.OP_NAME.get(i["opcode"]) == "SoftmaxXEntFwd"][-1]
    return ins["inp"][3], ins["out"][0], ins["out"][1]


def py_evaluate(eng, oset, plan):
    """EvaluateMetrics driven from Python (update_engine.cc:557-650)."""
    h = plan.header
    pos = oset.serving_pos()
    oset.cursor = 0
    rows_per = h["seq_len"] if h["input_kind"] == 1 else 1
    per_step = h["batch"] // rows_per
    batches = max(1, -(-oset.num_samples // per_step))
    pref, _, cols = eval_probs(plan)
    total, hits, counted = 0.0, 0, 0
    for b in range(batches):
        x, lab = oset.fill_batch(h["batch"])
        xa = np.frombuffer(x, np.int32 if h["input_kind"] == 1 else f32)
        la = np.frombuffer(lab, np.int32)
        eng.stage(xa, la)
        eng.run(PROGRAM_EVAL)
        total += eng.loss()
        real = min(per_step, max(oset.num_samples - b * per_step, 0)) * rows_per
        probs = eng.read(pref, h["batch"] * cols).reshape(h["batch"], cols)
        hits += fo.argmax_hits(probs[:real], la[:real])
        counted += real
    oset.restore_serving_pos(*pos)
    return float(f32(total / batches)), float(f32(hits / counted))


def window_means(curve, steps):
    w = max(1, min(20, steps // 5))
    first = float(f32(np.sum(np.asarray(curve[:w], np.float64)) / w))
    last = float(f32(np.sum(np.asarray(curve[steps - w:], np.float64)) / w))
    return first, last


def check_runner(plan, make_native, make_oracle, steps, shuffle_seed):
    ds = make_native()
    val = ds.split_validation(0.2)
    ds.enable_shuffle(shuffle_seed)
    e1 = DeviceUpdateEngine(plan.blob)
    rep = e1.train_dataset(ds, steps=steps, validation=val)

    o = make_oracle()
    ov = o.split_validation(0.2)
    o.enable_shuffle(shuffle_seed)
    e2 = DeviceUpdateEngine(plan.blob)
    h = plan.header
    v0 = py_evaluate(e2, ov, plan)
    curve = []
    for _ in range(steps):
        x, lab = o.fill_batch(h["batch"])
        xa = np.frombuffer(x, np.int32 if h["input_kind"] == 1 else f32)
        curve.append(e2.train_step(xa, np.frombuffer(lab, np.int32)))
    v1 = py_evaluate(e2, ov, plan)
    curve = np.array(curve, f32)

    assert rep["steps"] == steps
    assert np.array_equal(rep["loss_curve"].view(np.uint32), curve.view(np.uint32))
    assert rep["has_validation"] and rep["has_val_accuracy"]
    assert (rep["val_initial_loss"], rep["val_initial_accuracy"]) == pytest.approx(v0, abs=0)
    assert (rep["val_final_loss"], rep["val_final_accuracy"]) == pytest.approx(v1, abs=0)
    first, last = window_means(curve, steps)
    assert rep["initial_avg_loss"] == first and rep["final_avg_loss"] == last
    assert rep["improved"] == (v1[0] < v0[0])
    # pipelining is invisible: the feeder stands exactly after the consumed batches
    assert ds.serving_pos() == o.serving_pos()
    # and the parameters match bit for bit
    for _, ref, _, n in plan.params:
        assert np.array_equal(e1.read(ref, n).view(np.uint32), e2.read(ref, n).view(np.uint32))
    m = e1.evaluate_metrics(val)
    assert (m["loss"], m["accuracy"]) == pytest.approx(py_evaluate(e2, ov, plan), abs=0)
    e1.close()
    e2.close()


def test_train_and_evaluate_feature_rows_c1(torch_dev):
    w = configs.make("c1")
    plan = planner.compile_update(w.model, w.cfg)
    rng = np.random.default_rng(21)
    n = 230  # not a multiple of the batch: the eval pass wraps its last batch
    X = rng.standard_normal((n, 256)).astype(f32)
    y = rng.integers(0, 256, n).astype(np.int32).tobytes()
    check_runner(plan, lambda: feeder.Dataset.from_memory(X, y, n, 256, 1),
                 lambda: fo.Dataset.from_memory(X, y, n, 256, 1, 0), steps=23, shuffle_seed=11)


def test_train_and_evaluate_token_records_c3s(torch_dev):
    w = configs.make("c3s")
    plan = planner.compile_update(w.model, w.cfg)
    h = plan.header
    seq = h["seq_len"]
    rng = np.random.default_rng(3)
    records = 3 * (h["batch"] // seq) + 1
    toks = configs.zipf_tokens(rng, w.vocab, records * (seq + 1)).astype(np.int32)
    check_runner(plan, lambda: feeder.Dataset.from_tokens(toks, records, seq),
                 lambda: fo.Dataset.from_tokens(toks, records, seq), steps=5, shuffle_seed=2)


def test_timed_launches_survive_an_evaluation(torch_dev):
    """Launches marked for timing stay marked, and timed, across an
    evaluation that allocates the accuracy buffers: the train graph keeps
    its stamp nodes and its results are those of an unmarked engine."""
    w = configs.make("c1")
    plan = planner.compile_update(w.model, w.cfg)
    gemms = [i for i, ins in enumerate(plan.train)
             if planner.OP_NAME[ins["opcode"]] in ("GemmNN", "GemmNT")]
    rng = np.random.default_rng(5)
    n = 96
    X = rng.standard_normal((n, 256)).astype(f32)
    y = rng.integers(0, 256, n).astype(np.int32).tobytes()
    runs = []
    for mark in (False, True):
        e = DeviceUpdateEngine(plan.blob)
        if mark:
            e.mark_timed(0, gemms)
        x0, y0 = configs.batch(w, 0)
        losses = [e.train_step(x0, y0)]
        m = e.evaluate_metrics(feeder.Dataset.from_memory(X, y, n, 256, 1))
        x1, y1 = configs.batch(w, 1)
        losses.append(e.train_step(x1, y1))
        if mark:
            t = e.marked_times(0)
            assert t.shape == (len(gemms),) and np.all(t > 0) and np.all(t < 100.0)
        runs.append((np.array(losses, f32), m["loss"], m["accuracy"]))
        e.close()
    assert np.array_equal(runs[0][0].view(np.uint32), runs[1][0].view(np.uint32))
    assert runs[0][1:] == runs[1][1:]


def test_train_rejects_mismatched_dataset(torch_dev):
    w = configs.make("c1")
    plan = planner.compile_update(w.model, w.cfg)
    e = DeviceUpdateEngine(plan.blob)
    bad = feeder.Dataset.from_memory(np.zeros(10 * 255, f32), np.zeros(10, np.int32).tobytes(),
                                     10, 255, 1)
    with pytest.raises(RuntimeError, match="UpdateEngine: dataset input width does not match"):
        e.train_dataset(bad, steps=1)
    toks = feeder.Dataset.from_tokens(np.arange(9, dtype=np.int32), 1, 8)
    with pytest.raises(RuntimeError, match="takes feature rows, but the dataset carries token ids"):
        e.evaluate_metrics(toks)
    e.close()


def _ten_sample_set(seed=42):
    """Ten class-labelled feature rows under a shuffled feeder: every
    32-row batch of C1 wraps several epochs, so a resumed serving position
    must replay reshuffles, not just a cursor."""
    rng = np.random.default_rng(5)
    X = rng.standard_normal(10 * 256).astype(f32)
    y = rng.integers(0, 256, 10).astype(np.int32).tobytes()
    ds = feeder.Dataset.from_memory(X, y, 10, 256, 1)
    ds.enable_shuffle(seed)
    return ds


def test_resumed_run_matches_uninterrupted_run_bitwise(torch_dev, tmp_path):
    """update_engine_test.cc:402-444: six uninterrupted steps, against three
    steps, a checkpoint, a cold engine and feeder, and a resume for three
    more: the same run, bit for bit (the persistent segment and step_)."""
    w = configs.make("c1")
    plan = planner.compile_update(w.model, w.cfg)
    n = plan.header["persistent_size"] // 4
    straight = DeviceUpdateEngine(plan.blob)
    straight.train_dataset(_ten_sample_set(), steps=6)
    ck = str(tmp_path / "ck.sekp")
    first = DeviceUpdateEngine(plan.blob)
    first.train_dataset(_ten_sample_set(), steps=3)
    first.save_checkpoint(ck)
    first.close()
    resumed = DeviceUpdateEngine(plan.blob)
    resumed.train_dataset(_ten_sample_set(), steps=3, checkpoint_path=ck, resume=True)
    assert straight.step == 6 and resumed.step == 6
    assert np.array_equal(straight.read(0, n).view(np.uint32), resumed.read(0, n).view(np.uint32))
    straight.close()
    resumed.close()


def test_checkpoint_restores_step_and_state(torch_dev, tmp_path):
    """update_engine_test.cc:380-400: a load after further training puts
    step_ and the persistent segment back; periodic checkpoints
    (checkpoint_every) hold the step they were taken at; a checkpoint of
    another plan is refused and leaves the arena alone."""
    w = configs.make("c1")
    plan = planner.compile_update(w.model, w.cfg)
    n = plan.header["persistent_size"] // 4
    e = DeviceUpdateEngine(plan.blob)
    ck = str(tmp_path / "ck.sekp")
    e.train_dataset(_ten_sample_set(), steps=3)
    e.save_checkpoint(ck)
    saved = e.read(0, n)
    e.train_dataset(_ten_sample_set(), steps=4)
    assert e.step == 7
    e.load_checkpoint(ck)
    assert e.step == 3
    assert np.array_equal(e.read(0, n).view(np.uint32), saved.view(np.uint32))
    periodic = str(tmp_path / "every2.sekp")
    e.train_dataset(_ten_sample_set(), steps=5, checkpoint_path=periodic, checkpoint_every=2)
    assert e.step == 8
    from seeml_amd import _lib
    err = C.create_string_buffer(256)
    dst = (C.c_uint8 * (4 * n))()
    step = C.c_uint64()
    assert _lib.lib().seeml_hip_checkpoint_read(periodic.encode(), plan.header["plan_hash"], 4 * n,
                                                dst, C.byref(step), err, 256) == 0
    assert step.value == 8
    other = planner.compile_update(w.model, planner.UpdateConfig(**{**w.cfg.__dict__, "lr": 2e-3}))
    o = DeviceUpdateEngine(other.blob)
    before = o.read(0, n)
    with pytest.raises(RuntimeError, match="Checkpoint: checkpoint belongs to a different plan"):
        o.load_checkpoint(ck)
    assert np.array_equal(o.read(0, n).view(np.uint32), before.view(np.uint32)) and o.step == 0
    o.close()
    e.close()


def test_should_stop_interrupts_and_the_loss_curve_records(torch_dev):
    """update_engine_test.cc:730-745: should_stop polled once per step; the
    26th poll stops a 400-step run after 25 steps, with stopped_early set,
    25 recorded losses, and the state of a plain 25-step run."""
    w = configs.make("c1")
    plan = planner.compile_update(w.model, w.cfg)
    n = plan.header["persistent_size"] // 4
    polled = [0]

    def stop():
        polled[0] += 1
        return polled[0] > 25

    e = DeviceUpdateEngine(plan.blob)
    rep = e.train_dataset(_ten_sample_set(), steps=400, should_stop=stop)
    assert rep["stopped_early"] and rep["steps"] == 25 and polled[0] == 26
    assert len(rep["loss_curve"]) == 25 and e.step == 25
    plain = DeviceUpdateEngine(plan.blob)
    rep2 = plain.train_dataset(_ten_sample_set(), steps=25)
    assert not rep2["stopped_early"]
    assert np.array_equal(rep["loss_curve"].view(np.uint32), rep2["loss_curve"].view(np.uint32))
    assert np.array_equal(e.read(0, n).view(np.uint32), plain.read(0, n).view(np.uint32))
    e.close()
    plain.close()


def test_concurrent_engines_on_one_gpu_equal_their_serial_runs(torch_dev):
    """update_system_test.cc:784-822: two engines training at once from two
    host threads — each with its own arena, stream, graph and feeder, on
    the one GPU — each end bit for bit where its serial run ends."""
    import threading

    def make(name):
        w = configs.make(name)
        return w, planner.compile_update(w.model, w.cfg)

    jobs = [make("c3s"), make("c4m")]

    def dataset(w, seed):
        seq = w.seq
        records = 3 * (w.cfg.batch // seq) + 1
        toks = configs.zipf_tokens(np.random.default_rng(seed), w.vocab,
                                   records * (seq + 1)).astype(np.int32)
        ds = feeder.Dataset.from_tokens(toks, records, seq)
        ds.enable_shuffle(seed)
        return ds

    def run(k, out):
        w, plan = jobs[k]
        e = DeviceUpdateEngine(plan.blob)
        rep = e.train_dataset(dataset(w, 40 + k), steps=12)
        out[k] = (rep["loss_curve"].copy(), e.read(0, plan.header["persistent_size"] // 4))
        e.close()

    serial = [None, None]
    run(0, serial)
    run(1, serial)
    threaded = [None, None]
    ts = [threading.Thread(target=run, args=(k, threaded)) for k in range(2)]
    for t in ts:
        t.start()
    for t in ts:
        t.join()
    for k in range(2):
        assert threaded[k] is not None, k
        for a, b in zip(threaded[k], serial[k]):
            assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), k
