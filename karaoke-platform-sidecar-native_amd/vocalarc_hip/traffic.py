"""HBM traffic of the dominant kernel from rocprofv3 counter runs.

Two `rocprofv3 --pmc` runs of `python -m vocalarc_hip.kernel_bench --only copy,ff1`
(one with FETCH_SIZE, one with WRITE_SIZE) give KiB per dispatch for the
FFN up-projection GEMM (fp32 on fp16 matrix cores by two-piece operand splitting) at
the 8-window pass shape and for a plain device copy
of 1.27 GB.  Each counter is scaled by what it reads for the copy (known
bytes read and written), and the result is written as a short summary:

    python -m vocalarc_hip.traffic FETCH_DIR WRITE_DIR OUT.md "<commands>"
"""

from __future__ import annotations

import csv
import statistics
import sys
from pathlib import Path

COPY_BYTES = 496 * 801 * 801 * 4          # read once and written once by the copy
GEMM_KERNEL = "gemm_h2_kernel<4, true, false, false>"  # GELU-GLU epilogue, A as h2 rows: the FFN up-projection
COPY_KERNEL = "__amd_rocclr_copyBuffer"  # torch copy_ of a contiguous tensor is a runtime blit
# A as h2 rows (the bytes of fp32), W as two fp16 planes, bias fp32, output fp32
FF1_ALGORITHMIC = 397296 * 384 * 4 + 2 * 3072 * 384 * 2 + 3072 * 4 + 397296 * 1536 * 4


def _per_dispatch(run_dir: str, counter: str, needle: str, grid: int | None = None) -> float:
    path = next(Path(run_dir).rglob("*counter_collection.csv"))
    vals = []
    for r in csv.DictReader(open(path)):
        if r["Counter_Name"] == counter and needle in r["Kernel_Name"]:
            if grid is None or int(r["Grid_Size"]) == grid:
                vals.append(float(r["Counter_Value"]))
    if not vals:
        raise SystemExit(f"no {counter} rows for {needle} in {path}")
    return statistics.median(vals)


def main() -> int:
    fetch_dir, write_dir, out, commands = sys.argv[1:5]
    ff1_grid = 1552 * 24 * 512  # row tiles x column tiles x threads per workgroup
    f_copy = _per_dispatch(fetch_dir, "FETCH_SIZE", COPY_KERNEL) * 1024
    w_copy = _per_dispatch(write_dir, "WRITE_SIZE", COPY_KERNEL) * 1024
    f_gemm = _per_dispatch(fetch_dir, "FETCH_SIZE", GEMM_KERNEL, ff1_grid) * 1024
    w_gemm = _per_dispatch(write_dir, "WRITE_SIZE", GEMM_KERNEL, ff1_grid) * 1024
    kf, kw = COPY_BYTES / f_copy, COPY_BYTES / w_copy
    traffic = f_gemm * kf + w_gemm * kw
    lines = [
        "# HBM traffic of the FFN up-projection GEMM (GELU-GLU epilogue), one 8-window pass",
        "", "Commands (repository root, MI355X box):", "", "```", commands.strip(), "```", "",
        f"* copy calibration (1.27 GB read + 1.27 GB written): FETCH_SIZE {f_copy / 1e9:.4f} GB, WRITE_SIZE {w_copy / 1e9:.4f} GB"
        f" -> factors {kf:.4f} (fetch), {kw:.4f} (write)",
        f"* GEMM M=397296 K=384 N=3072 (median per dispatch): FETCH_SIZE {f_gemm / 1e9:.4f} GB, WRITE_SIZE {w_gemm / 1e9:.4f} GB",
        f"* calibrated traffic per launch: {traffic / 1e9:.4f} GB "
        f"(algorithmic: {FF1_ALGORITHMIC / 1e9:.4f} GB = A 610.3 MB + W planes 4.7 MB + output 2440.6 MB)",
        "", f"traffic_bytes_per_launch: {int(traffic)}",
    ]
    Path(out).write_text("\n".join(lines) + "\n")
    print("\n".join(lines))
    return 0


if __name__ == "__main__":
    sys.exit(main())
