"""LDS bank-conflict cost of 128-bit access patterns (one wavefront each).

    rocprofv3 --pmc SQ_LDS_BANK_CONFLICT SQ_INSTS_LDS SQ_LDS_IDX_ACTIVE --output-format csv \\
        -d gpurun_out/lds -o run -- python3 -u -m compact_amd.bench_lds > gpurun_out/lds.log
    python3 -m compact_amd.bench_lds --summarize gpurun_out/lds/run_counter_collection.csv \\
        gpurun_out/lds.log

The first command dispatches cpt_probe_lds_pattern once per pattern (1024 blocks x 2000
accesses) and prints the pattern names in dispatch order; the second joins the per-dispatch
counters with those names and prints conflict cycles per LDS instruction next to the lane-group
model below.

Patterns:
- the GEMM engine's K-major layout (row r at r * 64 + (r / 2) * 8 elements, 8-element chunks):
  the 32x32x16 fragment read (lane l: row l % 32, chunk l / 32), a 16x16x32 fragment read
  (row l % 16, chunk l / 16) and the stores (row l / 8, chunk l % 8);
- a layout made for the 16x16x32 read: 64-element rows, chunk XOR (row & 6);
- pair tests: lane l at byte 16 l (every 16-lane set covers the 64 banks once), then lane j
  moved onto lane i's banks at another address. A conflict means i and j share a cycle;
- 64-bit reads, plain and transposing (ds_read_b64_tr_b16), at the engine's MN-major fragment
  addresses (rows 288 elements apart, and 256 for comparison) and lane-linear.

Lane-group model for reads (fits every read pattern measured): a 128-bit read takes 4 cycles
serving lanes {0-7, 24-31}, {8-15, 16-23}, {32-39, 56-63} and {40-47, 48-55}.  A 128-bit write
takes about 8 cycles (8 lanes each); its grouping is not pinned down (the pair tests put lane 0
with lanes 1-4, 12, 13 and 15 or with their bank partners 16 lanes apart, and never with 8, 16,
24 or 32), so writes get no model column.
"""

from __future__ import annotations

import argparse
import collections
import csv

READ_GROUPS = [list(range(0, 8)) + list(range(24, 32)), list(range(8, 24)),
               list(range(32, 40)) + list(range(56, 64)), list(range(40, 56))]


def model_conflicts(offs: list[int]) -> int:
    """Extra cycles a read pattern costs under the lane-group model: per group,
    the largest number of distinct dwords that fall on one of the 64 banks,
    minus 1."""
    extra = 0
    for g in READ_GROUPS:
        banks: dict[int, set[int]] = {}
        for lane in g:
            for w in range(4):
                dw = offs[lane] // 4 + w
                banks.setdefault(dw % 64, set()).add(dw)
        extra += max(len(v) for v in banks.values()) - 1
    return extra


def _engine(r: int, c: int) -> int:
    return (r * 64 + (r >> 1) * 8 + c * 8) * 2


def _swz(r: int, c: int) -> int:
    return (r * 64 + ((c ^ (r & 6)) * 8)) * 2


def patterns() -> dict[str, tuple[int, list[int]]]:
    """name -> (mode, byte offset per lane); mode False / True: 128-bit read /
    write, 2: ds_read_b64, 3: ds_read_b64_tr_b16."""
    pat: dict[str, tuple[int, list[int]]] = {}
    for name, f in (("engine layout", _engine), ("16x16 layout", _swz)):
        pat[f"{name}: 32x32x16 fragment read"] = (False, [f(l & 31, l >> 5) for l in range(64)])
        pat[f"{name}: 16x16x32 fragment read, k 0-31"] = (False, [f(l & 15, l >> 4) for l in range(64)])
        pat[f"{name}: 16x16x32 fragment read, k 32-63"] = (False, [f(l & 15, (l >> 4) + 4)
                                                                  for l in range(64)])
        pat[f"{name}: stores"] = (True, [f(l >> 3, l & 7) for l in range(64)])
    # 64-bit reads (mode 2 plain, 3 transposing): the engine's MN-major fragment read,
    # lane l at k-row 8 (l / 32) + (l % 16) / 4, mn 16 ((l / 16) % 2) + 4 (l % 4) of a
    # [64 k][LDM] tile, LDM 288 (the engine) or 256 (no row skew)
    for ldm in (288, 256):
        mn = [((8 * (l >> 5) + ((l & 15) >> 2)) * ldm + 16 * ((l >> 4) & 1) + 4 * (l & 3)) * 2
              for l in range(64)]
        pat[f"MN-major fragment, LDM {ldm}: ds_read_b64_tr_b16"] = (3, mn)
        pat[f"MN-major fragment, LDM {ldm}: ds_read_b64"] = (2, mn)
    pat["lane-linear ds_read_b64"] = (2, [8 * l for l in range(64)])
    pat["lane-linear ds_read_b64_tr_b16"] = (3, [8 * l for l in range(64)])
    pat["lane-linear read"] = (False, [16 * l for l in range(64)])
    pat["lane-linear write"] = (True, [16 * l for l in range(64)])
    for write in (False, True):
        pairs = [(0, 1), (0, 7), (0, 8), (0, 15), (0, 16), (0, 23), (0, 24), (0, 31), (0, 32), (0, 33),
                 (8, 16), (8, 24), (16, 24), (32, 56), (40, 48), (40, 56)]
        if write:
            pairs = [(0, 1), (0, 2), (0, 3), (0, 4), (0, 8), (0, 12), (0, 13), (0, 15), (0, 16), (0, 24),
                     (0, 32), (4, 8), (4, 11), (8, 16), (16, 20), (16, 28), (32, 44), (36, 40)]
        for i, j in pairs:
            o = [16 * l for l in range(64)]
            o[j] = 16 * i + 8192
            pat[f"pair {i},{j} {'write' if write else 'read'}"] = (write, o)
    return pat


def run(iters: int = 2000, blocks: int = 1024):
    import torch
    from . import _lib
    from ._lib import check
    lib = _lib.lib()
    out = torch.empty(blocks * 64, device="cuda")
    for name, (write, offs) in patterns().items():
        align = 8 if write >= 2 else 16
        assert len(offs) == 64 and all(0 <= o <= 0xfff8 and o % align == 0 for o in offs), name
        t = torch.tensor(offs, dtype=torch.int32, device="cuda")
        print(f"dispatch {name}", flush=True)
        check(lib.cpt_probe_lds_pattern(t.data_ptr(), int(write), blocks, iters, out.data_ptr(),
                                        torch.cuda.current_stream().cuda_stream), "probe_lds_pattern")
        torch.cuda.synchronize()
    print("done", flush=True)


def summarize(csv_path: str, log_path: str):
    per: dict[int, dict[str, float]] = collections.defaultdict(dict)
    for r in csv.DictReader(open(csv_path)):
        if "lds_pattern_kernel" in r["Kernel_Name"]:
            per[int(r["Dispatch_Id"])][r["Counter_Name"]] = float(r["Counter_Value"])
    names = [ln.split("dispatch ", 1)[1].strip() for ln in open(log_path) if ln.startswith("dispatch ")]
    pat = patterns()
    print("| pattern | conflict cycles / instruction | LDS active cycles / instruction | read model |")
    print("|---|---|---|---|")
    for (_, c), name in zip(sorted(per.items()), names):
        n = c["SQ_INSTS_LDS"]
        write, offs = pat[name]
        print(f"| {name} | {c['SQ_LDS_BANK_CONFLICT'] / n:.2f} | {c['SQ_LDS_IDX_ACTIVE'] / n:.2f} | "
              f"{model_conflicts(offs) if write is False else '-'} |")


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--summarize", nargs=2, metavar=("CSV", "LOG"))
    a = ap.parse_args()
    if a.summarize:
        summarize(*a.summarize)
    else:
        run()


if __name__ == "__main__":
    main()
