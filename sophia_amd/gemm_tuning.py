"""Selection of library GEMM kernels for the decoder's projections.

The token-parallel projections of the hybrid decoder (the fused KDA input
projection, SiTU-GLU up/down, o_proj, MLA's down/up projections, the head)
are plain GEMMs and run on hipBLASLt / rocBLAS through torch.  Their default
heuristics pick a kernel per shape; torch's TunableOp can instead time the
candidate solutions once and keep the fastest per shape in a CSV file.  The
file shipped beside this module holds that choice for the shapes of the
1,536-wide decoder on gfx950 (16,624-token mixed step); its header records the
torch, HIP, hipBLASLt and rocBLAS versions it is valid for, and TunableOp
ignores it if they differ.  Shapes not in the file keep the default heuristic.

Regenerate it on an MI355X with ``python bench.py --only mixed --no-cpu
--tune-gemms sophia_amd/gemm_tuning_gfx950.csv``.
"""

from __future__ import annotations

import os

DEFAULT_FILE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "gemm_tuning_gfx950.csv")


def use_tuned_gemms(path: str = DEFAULT_FILE, *, tune: bool = False,
                    max_tuning_ms: int = 100) -> bool:
    """Route torch's GEMMs through TunableOp with the selections in ``path``.

    tune=False: only read the file (no timing runs); returns whether it was
    read.  tune=True: shapes missing from the file are timed on first use
    (up to ``max_tuning_ms`` per candidate) and the file is rewritten with
    them when the process ends."""
    import torch.cuda.tunable as tunable

    tunable.enable(True)
    tunable.tuning_enable(bool(tune))
    if tune:
        tunable.set_max_tuning_duration(int(max_tuning_ms))
    tunable.set_filename(path)
    return bool(os.path.exists(path) and tunable.read_file(path))


def use_default_gemms() -> None:
    """Back to the libraries' own per-shape heuristics."""
    import torch.cuda.tunable as tunable

    tunable.tuning_enable(False)
    tunable.enable(False)
