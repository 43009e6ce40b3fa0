"""Summarise a rocprofv3 --kernel-trace CSV by (kernel, launch grid).

Grouping by the grid as well as the name separates the different GEMM
shapes that share one kernel template. Usage:
    python tests/perf/trace_summary.py <..._kernel_trace.csv> [top_n]
"""
import collections
import csv
import re
import sys


def short(name: str) -> str:
    name = re.sub(r"seeml_hip::\(anonymous namespace\)::", "", name)
    name = re.sub(r"\(.*\)$", "", name)
    return name.replace("void ", "")


def main(path, top=25):
    groups = collections.defaultdict(list)
    for r in csv.DictReader(open(path)):
        key = (short(r["Kernel_Name"]),
               f'{r["Grid_Size_X"]}x{r["Grid_Size_Y"]}x{r["Grid_Size_Z"]}',
               r["VGPR_Count"], r["Accum_VGPR_Count"], r["LDS_Block_Size"])
        groups[key].append(int(r["End_Timestamp"]) - int(r["Start_Timestamp"]))
    total = sum(sum(v) for v in groups.values())
    rows = sorted(groups.items(), key=lambda kv: -sum(kv[1]))
    print(f"{'kernel':62s} {'grid(work-items)':>18s} {'calls':>5s} {'avg_us':>9s} "
          f"{'med_us':>9s} {'min_us':>8s} {'share':>6s}  vgpr/agpr/lds")
    for (name, grid, vg, ag, lds), d in rows[:top]:
        med = sorted(d)[len(d) // 2]
        print(f"{name[:62]:62s} {grid:>18s} {len(d):5d} {sum(d) / len(d) / 1e3:9.2f} "
              f"{med / 1e3:9.2f} {min(d) / 1e3:8.2f} {sum(d) / total:6.1%}  {vg}/{ag}/{lds}")


if __name__ == "__main__":
    main(sys.argv[1], int(sys.argv[2]) if len(sys.argv) > 2 else 25)
