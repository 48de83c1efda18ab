"""Summaries of rocprofv3 result databases (rocpd SQLite) for the profiles/ directory.

  python -m helios_glm53flash_amd.profiling stats <kernel-trace.db>
      per-kernel dispatch count and average / min / max duration (us)
  python -m helios_glm53flash_amd.profiling traffic <fetch.db> <write.db> [--cmd "..."]
      HBM bytes per launch of the MoE decode layer kernel from FETCH_SIZE and WRITE_SIZE passes, each
      scaled by what the same counter reads for the calibration copy (256 MiB read + 256 MiB write)
      of bench.py --profile-only
  python -m helios_glm53flash_amd.profiling counters <pmc.db> <kernel-name-part>
      mean value per dispatch of each counter collected for the matching kernels
  python -m helios_glm53flash_amd.profiling utilisation <kernel-name-part> <pmc.db>...
      per-dispatch utilisation of the matrix cores, VALU and LDS from the passes' counters (see
      utilisation() for the definitions)
"""
from __future__ import annotations

import json
import sqlite3
import sys

COPY_BYTES = 256 << 20


def kernel_stats(db: str) -> list[dict]:
    c = sqlite3.connect(db)
    rows = c.execute("select name, count(*), avg(end-start), min(end-start), max(end-start) from kernels "
                     "group by name order by sum(end-start) desc").fetchall()
    return [{"kernel": n, "calls": k, "avg_us": a / 1e3, "min_us": lo / 1e3, "max_us": hi / 1e3}
            for n, k, a, lo, hi in rows]


def counter_means(db: str, counter: str) -> dict[str, float]:
    c = sqlite3.connect(db)
    rows = c.execute("select kernel_name, avg(value) from counters_collection where counter_name = ? "
                     "group by kernel_name", (counter,)).fetchall()
    return {n: v for n, v in rows}


def calibration_value(db: str, counter: str) -> float:
    """Counter value of the 256 MiB calibration copy: the largest copy dispatch of the run (the
    runtime's blit kernel also serves the small host transfers, which read far less)."""
    c = sqlite3.connect(db)
    (v,) = c.execute("select max(value) from counters_collection where counter_name = ? and "
                     "kernel_name like '%copy%'", (counter,)).fetchone()
    return float(v)


def _pick(d: dict[str, float], key: str) -> float:
    vals = [v for n, v in d.items() if key in n]
    if not vals:
        raise KeyError(key)
    return sum(vals) / len(vals)


def traffic(fetch_db: str, write_db: str, cmd: str = "") -> dict:
    f = counter_means(fetch_db, "FETCH_SIZE")
    w = counter_means(write_db, "WRITE_SIZE")
    copy_f = calibration_value(fetch_db, "FETCH_SIZE")
    copy_w = calibration_value(write_db, "WRITE_SIZE")
    kf = COPY_BYTES / (copy_f * 1024.0)   # bytes per reported KiB, read side
    kw = COPY_BYTES / (copy_w * 1024.0)
    out = {"command": cmd, "copy_calibration": {"bytes": COPY_BYTES, "FETCH_SIZE_KiB": copy_f,
                                                "WRITE_SIZE_KiB": copy_w, "read_scale": kf, "write_scale": kw},
           "kernels": {}}
    for phase, key in (("moe_decode", "moe_decode_kernel"),):
        fk, wk = _pick(f, key), _pick(w, key)
        out["kernels"][phase] = {"FETCH_SIZE_KiB": fk, "WRITE_SIZE_KiB": wk,
                                 "read_bytes": fk * 1024 * kf, "write_bytes": wk * 1024 * kw,
                                 "hbm_bytes_per_launch": round(fk * 1024 * kf + wk * 1024 * kw)}
    return out


def counters(db: str, key: str) -> dict[str, float]:
    """Mean value per dispatch of every counter collected for the kernels whose name contains key."""
    c = sqlite3.connect(db)
    rows = c.execute("select counter_name, avg(value) from counters_collection where kernel_name like ? "
                     "group by counter_name", (f"%{key}%",)).fetchall()
    return {n: float(v) for n, v in rows}


# MI355X: 8 XCDs, 256 CUs, 4 SIMDs per CU.  GRBM_GUI_ACTIVE is summed over the XCDs (cycles of one
# XCD = value / 8); SQ_ACTIVE_INST_VALU counts in units of 4 cycles (a wave64 VALU instruction
# issues over 4 cycles); SQ_VALU_MFMA_BUSY_CYCLES is summed over the SIMDs; the LDS counters over
# the CUs.
XCDS, CUS, SIMDS = 8, 256, 1024


def utilisation(key: str, dbs: list[str]) -> dict[str, float]:
    c: dict[str, float] = {}
    for db in dbs:
        for k, v in counters(db, key).items():
            c.setdefault(k, v)
    cyc = c["GRBM_GUI_ACTIVE"] / XCDS
    out = {"cycles_per_xcd": cyc}
    if "SQ_VALU_MFMA_BUSY_CYCLES" in c:
        out["mfma_busy"] = c["SQ_VALU_MFMA_BUSY_CYCLES"] / (cyc * SIMDS)
    if "SQ_ACTIVE_INST_VALU" in c:
        out["valu_busy"] = 4 * c["SQ_ACTIVE_INST_VALU"] / (cyc * SIMDS)
    if "SQ_VALU_MFMA_COEXEC_CYCLES" in c:
        out["valu_mfma_coexec"] = c["SQ_VALU_MFMA_COEXEC_CYCLES"] / (cyc * SIMDS)
    if "SQ_LDS_IDX_ACTIVE" in c:
        out["lds_active"] = c["SQ_LDS_IDX_ACTIVE"] / (cyc * CUS)
    if "SQ_LDS_BANK_CONFLICT" in c:
        out["lds_bank_conflict"] = c["SQ_LDS_BANK_CONFLICT"] / (cyc * CUS)
    if "SQ_INSTS_VALU" in c and "SQ_INSTS_MFMA" in c:
        out["valu_per_mfma"] = c["SQ_INSTS_VALU"] / c["SQ_INSTS_MFMA"]
    if "SQ_INSTS_VALU_MFMA_MOPS_F16" in c:
        out["mfma_flops"] = 512.0 * c["SQ_INSTS_VALU_MFMA_MOPS_F16"]
    return {k: round(v, 4) if v < 100 else v for k, v in out.items()}


def main(argv: list[str]) -> None:
    if len(argv) >= 2 and argv[0] == "stats":
        for r in kernel_stats(argv[1]):
            print(f"{r['calls']:6d}  avg {r['avg_us']:10.3f} us  min {r['min_us']:10.3f}  max {r['max_us']:10.3f}  "
                  f"{r['kernel'][:110]}")
    elif len(argv) >= 3 and argv[0] == "counters":
        print(json.dumps(counters(argv[1], argv[2]), indent=1))
    elif len(argv) >= 3 and argv[0] == "utilisation":
        print(json.dumps(utilisation(argv[1], argv[2:]), indent=1))
    elif len(argv) >= 3 and argv[0] == "traffic":
        cmd = argv[argv.index("--cmd") + 1] if "--cmd" in argv else ""
        print(json.dumps(traffic(argv[1], argv[2], cmd), indent=1))
    else:
        print(__doc__)
        sys.exit(2)


if __name__ == "__main__":
    main(sys.argv[1:])
