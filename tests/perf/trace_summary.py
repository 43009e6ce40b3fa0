"""Summarise a rocprofv3 --kernel-trace CSV by (kernel, launch grid).

Grouping by the grid as well as the name separates the different GEMM
shapes that share one kernel template. Usage:
    python tests/perf/trace_summary.py <..._kernel_trace.csv> [top_n]
    python tests/perf/trace_summary.py <..._kernel_trace.csv> [top_n] --after-gap STEPS
With --after-gap, only the launches after the largest gap between kernel
starts count (graph_steps.py pauses before its timed steps), and calls and
times are per step.
"""
import collections
import csv
import re
import sys


def short(name: str) -> str:
    name = re.sub(r"seeml_hip::\(anonymous namespace\)::", "", name)
    name = re.sub(r"\(.*\)$", "", name)
    return name.replace("void ", "")


def main(path, top=25, steps=0):
    groups = collections.defaultdict(list)
    rows = list(csv.DictReader(open(path)))
    if steps:
        rows.sort(key=lambda r: int(r["Start_Timestamp"]))
        st = [int(r["Start_Timestamp"]) for r in rows]
        gap = max(range(1, len(st)), key=lambda i: st[i] - st[i - 1])
        rows = rows[gap:]
        span = int(rows[-1]["End_Timestamp"]) - int(rows[0]["Start_Timestamp"])
    for r in rows:
        key = (short(r["Kernel_Name"]),
               f'{r["Grid_Size_X"]}x{r["Grid_Size_Y"]}x{r["Grid_Size_Z"]}',
               r["VGPR_Count"], r["Accum_VGPR_Count"], r["LDS_Block_Size"])
        groups[key].append(int(r["End_Timestamp"]) - int(r["Start_Timestamp"]))
    total = sum(sum(v) for v in groups.values())
    if steps:
        print(f"{len(rows) / steps:.0f} launches per step, kernels busy {total / steps / 1e6:.3f} ms "
              f"of a {span / steps / 1e6:.3f} ms span per step")
        print(f"{'kernel':62s} {'grid(work-items)':>18s} {'per step':>8s} {'avg_us':>9s} "
              f"{'ms/step':>8s} {'share':>6s}  vgpr/agpr/lds")
        for (name, grid, vg, ag, lds), d in sorted(groups.items(), key=lambda kv: -sum(kv[1]))[:top]:
            print(f"{name[:62]:62s} {grid:>18s} {len(d) / steps:8.1f} {sum(d) / len(d) / 1e3:9.2f} "
                  f"{sum(d) / steps / 1e6:8.3f} {sum(d) / total:6.1%}  {vg}/{ag}/{lds}")
        return
    rows = sorted(groups.items(), key=lambda kv: -sum(kv[1]))
    print(f"{'kernel':62s} {'grid(work-items)':>18s} {'calls':>5s} {'avg_us':>9s} "
          f"{'med_us':>9s} {'min_us':>8s} {'share':>6s}  vgpr/agpr/lds")
    for (name, grid, vg, ag, lds), d in rows[:top]:
        med = sorted(d)[len(d) // 2]
        print(f"{name[:62]:62s} {grid:>18s} {len(d):5d} {sum(d) / len(d) / 1e3:9.2f} "
              f"{med / 1e3:9.2f} {min(d) / 1e3:8.2f} {sum(d) / total:6.1%}  {vg}/{ag}/{lds}")


if __name__ == "__main__":
    args = [a for a in sys.argv[1:]]
    steps = 0
    if "--after-gap" in args:
        k = args.index("--after-gap")
        steps = int(args[k + 1])
        del args[k:k + 2]
    main(args[0], int(args[1]) if len(args) > 1 else 25, steps)
