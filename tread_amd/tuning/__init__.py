"""GEMM solution tables for the projection GEMMs (hipBLASLt / rocBLAS through PyTorch TunableOp).

The decoder's GEMMs stay plain library GEMMs; TunableOp only chooses, per GEMM shape, which of the
installed hipBLASLt / rocBLAS solutions runs. `gemm_gfx950_qwen2.5-7b.csv` holds the choices measured
on MI355X for the 7B-shaped reuse workload (recompute rows at 20 % and 50 % of the doc tokens,
with and without the 32 query rows riding along, deviation rows, query rows, full-prefill rows);
TunableOp checks the file's torch / HIP / hipBLASLt / rocBLAS / arch stamps before using it.
Shapes missing from the table run the library default.
"""
import os
import tempfile
from pathlib import Path

import torch

TABLE_7B = Path(__file__).resolve().with_name("gemm_gfx950_qwen2.5-7b.csv")


def use_tuned_gemms(tables=(TABLE_7B,), tune=False, out_file=None, max_tuning_ms=15, max_iterations=20):
    """Route torch GEMMs through TunableOp with the given solution tables. With tune=True, shapes
    not in the tables are benchmarked on first use (a one-off cost per shape) and written to
    out_file; otherwise unknown shapes use the library default and nothing is written."""
    tun = torch.cuda.tunable
    tun.enable(True)
    tun.tuning_enable(bool(tune))
    if tune:
        tun.set_max_tuning_duration(max_tuning_ms)
        tun.set_max_tuning_iterations(max_iterations)
    # TunableOp may write its results at exit: keep that out of the working directory
    tun.set_filename(str(out_file) if (tune and out_file) else
                     str(Path(tempfile.gettempdir()) / f"tread_tunableop_{os.getpid()}.csv"))
    for t in tables:
        if t and Path(t).exists():
            tun.read_file(str(t))
