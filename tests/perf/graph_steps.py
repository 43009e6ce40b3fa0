"""Runs a bench config's train step as the timed bench does (autotuned,
graph replay), for kernel traces of the steps alone:

  python3 tests/perf/graph_steps.py c4 3

Autotune, three warm-up steps, a one-second pause, then N steps. Under
`rocprofv3 --kernel-trace`, the pause is the largest gap between kernel
starts, so `trace_summary.py --after-gap N` keeps exactly the N steps'
launches. A profiling harness beside the tests: the product never imports it.
"""
import os
import sys
import time

sys.path.insert(0, os.path.join(os.path.dirname(os.path.abspath(__file__)), "..", "..", "see-ml_amd"))


def main():
    import torch
    from seeml_amd import DeviceUpdateEngine, configs, planner
    cfg = sys.argv[1] if len(sys.argv) > 1 else "c4"
    n = int(sys.argv[2]) if len(sys.argv) > 2 else 3
    w = configs.make(cfg)
    plan = planner.compile_update(w.model, w.cfg)
    e = DeviceUpdateEngine(plan.blob)
    plan.blob = None
    e.autotune(16)
    dev = torch.device("cuda:0")
    bs = []
    for s in range(2):
        x, y = configs.batch(w, s)
        bs.append((torch.from_numpy(x).to(dev), torch.from_numpy(y).to(dev)))
    for s in range(3):
        e.train_step(*bs[s % 2])
    torch.cuda.synchronize()
    print(f"graph_steps: {cfg} warm", flush=True)
    time.sleep(1.0)
    t0 = time.perf_counter()
    for s in range(n):
        e.train_step(*bs[s % 2])
    torch.cuda.synchronize()
    print(f"graph_steps: {cfg} {n} steps, {(time.perf_counter() - t0) * 1e3 / n:.3f} ms/step", flush=True)
    e.close()


if __name__ == "__main__":
    main()
