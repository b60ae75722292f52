"""Guards on the gfx950 machine code of this build (our own objects, disassembled with the ROCm
LLVM tools; skipped when the build or the tools are absent).

The global -> LDS loads are inline assembly that writes M0 (the LDS base of the load) one
instruction before the load. LLVM reserves M0 and does not preserve it across an asm statement
that clobbers it, so the build is only correct while no compiler-generated instruction keeps a
value in M0 across such a load. These checks hold that, in every object that contains such loads:
  * the only writes of M0 are the asm's `s_mov_b32 m0, sN`, each followed by `s_nop 0` and the
    load (so M0 is never carried over from earlier code into a load);
  * no instruction class that reads M0 implicitly besides those loads appears: indirect register
    indexing (v_movrel*, s_movrel*, s_set_gpr_idx_*), s_sendmsg, ds_*addtid*, GWS, ordered
    count, parameter interpolation, LDS direct reads.
Objects without the loads leave M0 to the compiler and are not constrained.
"""

import re
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
BUILD = ROOT / "_build"
LLVM = Path("/opt/rocm/llvm/bin")
TOOLS = [LLVM / "llvm-objcopy", LLVM / "clang-offload-bundler", LLVM / "llvm-objdump"]
M0_READERS = re.compile(r"\b(v_movrel\w*|s_movrel\w*|s_set_gpr_idx_\w+|s_sendmsg\w*|ds_\w*addtid\w*|"
                        r"ds_gws\w*|ds_ordered_count|v_interp\w*|lds_direct|lds_param_load)\b")


def _disassemble(obj: Path, tmp: Path) -> list[str]:
    bundle, code = tmp / f"{obj.stem}.bundle", tmp / f"{obj.stem}.co"
    subprocess.run([str(TOOLS[0]), f"--dump-section=.hip_fatbin={bundle}", str(obj)], check=True,
                   capture_output=True)
    subprocess.run([str(TOOLS[1]), "--type=o", "--targets=hipv4-amdgcn-amd-amdhsa--gfx950",
                    f"--input={bundle}", f"--output={code}", "--unbundle"], check=True, capture_output=True)
    out = subprocess.run([str(TOOLS[2]), "-d", str(code)], check=True, capture_output=True, text=True).stdout
    return [line.split("//")[0].strip() for line in out.splitlines() if line.startswith("\t")]


def _objects():
    if not BUILD.is_dir() or not all(t.exists() for t in TOOLS):
        return []
    return sorted(BUILD.glob("*.o"))


@pytest.mark.skipif(not _objects(), reason="needs the in-tree build (_build/*.o) and the ROCm LLVM tools")
def test_m0_is_only_set_for_the_global_to_lds_loads(tmp_path):
    loads = 0
    for obj in _objects():
        try:
            insts = _disassemble(obj, tmp_path)
        except subprocess.CalledProcessError:
            continue  # a host-only object (no device code)
        if not any(ins.startswith("global_load_lds_") for ins in insts):
            continue
        for i, ins in enumerate(insts):
            assert not M0_READERS.search(ins), f"{obj.name}: instruction reading M0 implicitly: {ins}"
            if re.search(r"\bm0\b", ins):
                assert re.match(r"s_mov_b32 m0, s\d+$", ins), f"{obj.name}: unexpected use of M0: {ins}"
                assert insts[i + 1] == "s_nop 0" and insts[i + 2].startswith("global_load_lds_"), \
                    f"{obj.name}: M0 written without the load that uses it: {insts[i:i + 3]}"
            if ins.startswith("global_load_lds_") or re.match(r"buffer_load_\w+ .*\blds\b", ins):
                loads += 1
                assert i >= 2 and insts[i - 1] == "s_nop 0" and insts[i - 2].startswith("s_mov_b32 m0,"), \
                    f"{obj.name}: global -> LDS load without its own M0 write: {insts[i - 2:i + 1]}"
    assert loads > 0  # the attention kernels' K/V and Q/dO rings
