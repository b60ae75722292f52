"""The recorded TunableOp solution file (aspec_amd/tuning/head_gemms_gfx950.csv) is well formed:
validator lines first (PyTorch, HIP, hipBLASLt, rocBLAS versions and the gfx950 arch), then one
solution per GEMM shape, covering the three head GEMMs of the config-2 step."""

import csv
from pathlib import Path

FILE = Path(__file__).resolve().parents[1] / "aspec_amd" / "tuning" / "head_gemms_gfx950.csv"


def test_solution_file_is_well_formed():
    rows = [r for r in csv.reader(FILE.read_text().splitlines()) if r]
    validators = {r[1]: r[2] for r in rows if r[0] == "Validator"}
    assert {"PT_VERSION", "HIP_VERSION", "HIPBLASLT_VERSION", "GCN_ARCH_NAME", "ROCBLAS_VERSION"} <= set(validators)
    assert validators["GCN_ARCH_NAME"].startswith("gfx950")
    entries = [r for r in rows if r[0] != "Validator"]
    assert entries and all(len(r) == 4 and r[0].startswith("GemmTunableOp_BFloat16_") for r in entries)
    assert all(float(r[3]) > 0 for r in entries)
    shapes = {r[1] for r in entries}
    assert len(shapes) == len(entries)  # one solution per shape
    # draft logits, teacher table and head dgrad of the config-2 step (V = 32000, H = 4096)
    for shape in ("tn_32000_8192_4096_ld_4096_4096_32000", "tn_32000_4096_4096_ld_4096_4096_32000",
                  "tn_4096_8192_32000_ld_32000_32000_4096"):
        assert shape in shapes
