"""GEMM solution tables for the projection GEMMs (hipBLASLt / rocBLAS through PyTorch TunableOp).

The decoder's GEMMs stay plain library GEMMs; TunableOp only chooses, per GEMM shape, which of the
installed hipBLASLt / rocBLAS solutions runs. `gemm_gfx950_<model>.csv` holds the choices measured
on MI355X for that model's reuse workload (`bench.py --workload ... --retune`: recompute rows at
0 %, 20 % and 50 % of the doc tokens, with and without the 32 query rows riding along, deviation
rows, query rows, full-prefill rows): the 7B 32k, 1.5B 16k and 0.5B 8k workloads. TunableOp
checks the file's torch / HIP / hipBLASLt / rocBLAS / arch stamps before using it. Shapes missing
from the table run the library default.
"""
import os
import tempfile
from pathlib import Path

import torch

TABLE_7B = Path(__file__).resolve().with_name("gemm_gfx950_qwen2.5-7b.csv")


def table_for(model_name):
    """The committed solution table of a model preset (`tread_amd.model.preset` names), or None."""
    p = Path(__file__).resolve().with_name(f"gemm_gfx950_{model_name}.csv")
    return p if p.exists() else None


def table_validators(path):
    """The Validator lines (name -> value) a TunableOp table was stamped with."""
    out = {}
    for line in Path(path).read_text().splitlines():
        parts = line.split(",", 2)
        if len(parts) == 3 and parts[0] == "Validator":
            out[parts[1]] = parts[2]
    return out


def use_tuned_gemms(tables=(TABLE_7B,), tune=False, out_file=None, max_tuning_ms=15, max_iterations=20):
    """Route torch GEMMs through TunableOp with the given solution tables. With tune=True, shapes
    not in the tables are benchmarked on first use (a one-off cost per shape) and written to
    out_file; otherwise unknown shapes use the library default and nothing is written.

    Returns the status of each table: whether TunableOp accepted it (its torch / HIP / hipBLASLt /
    rocBLAS / arch stamps match this process; otherwise every GEMM silently runs the library
    default), how many solutions are in effect, and which stamps differ."""
    tun = torch.cuda.tunable
    tun.enable(True)
    tun.tuning_enable(bool(tune))
    if tune:
        tun.set_max_tuning_duration(max_tuning_ms)
        tun.set_max_tuning_iterations(max_iterations)
    # TunableOp may write its results at exit: keep that out of the working directory
    tun.set_filename(str(out_file) if (tune and out_file) else
                     str(Path(tempfile.gettempdir()) / f"tread_tunableop_{os.getpid()}.csv"))
    status = []
    for t in tables:
        if not t or not Path(t).exists():
            status.append({"table": str(t), "loaded": False, "solutions": 0, "mismatched": ["missing file"]})
            continue
        ok = bool(tun.read_file(str(t)))
        have = dict(tun.get_validators())
        want = table_validators(t)
        mismatched = sorted(k for k, v in want.items() if k in have and have[k] != v)
        n = len(tun.get_results())
        status.append({"table": Path(t).name, "loaded": ok and not mismatched and n > 0, "solutions": n,
                       "mismatched": mismatched})
    return status
