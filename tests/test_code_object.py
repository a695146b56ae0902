"""The built library's gfx950 code objects (read from this build's own
.hip_fatbin section: one offload bundle per source file): no kernel uses
scratch memory except the fused forward + prune, whose site-program
interpreter's 32 registers do not fit beside the forward's. A kernel that starts spilling (a helper no longer
inlined, an array indexed at run time) shows up here before a benchmark
shows it: the streaming forward once went from 27 to 107 us that way."""

from __future__ import annotations

import re
import subprocess
from pathlib import Path

import pytest

from plastax_amd import _lib

LLVM = Path("/opt/rocm/llvm/bin")
ALLOWED = re.compile(r"k_forwardILi\dELb1E")  # k_forward<M, PRUNE=true>


def _kernels(tmp_path: Path) -> dict[str, dict[str, int]]:
    tools = [LLVM / "llvm-objcopy", LLVM / "clang-offload-bundler", LLVM / "llvm-readelf"]
    if not all(t.exists() for t in tools) or not Path(_lib.LIB_PATH).exists():
        pytest.skip("ROCm LLVM tools or the built library missing")
    fat = tmp_path / "fat.bin"
    subprocess.run([str(tools[0]), f"--dump-section=.hip_fatbin={fat}", str(_lib.LIB_PATH)], check=True,
                   capture_output=True)
    data = fat.read_bytes()
    magic = b"__CLANG_OFFLOAD_BUNDLE__"
    starts = [i for i in range(len(data)) if data.startswith(magic, i)] if magic in data else []
    assert starts, "no offload bundle in .hip_fatbin"
    notes = ""
    for j, a in enumerate(starts):
        end = starts[j + 1] if j + 1 < len(starts) else len(data)
        part, co = tmp_path / f"b{j}.bin", tmp_path / f"co{j}.elf"
        part.write_bytes(data[a:end])
        subprocess.run([str(tools[1]), "--type=o", f"--input={part}",
                        "--targets=hipv4-amdgcn-amd-amdhsa--gfx950", f"--output={co}", "--unbundle"], check=True,
                       capture_output=True)
        notes += subprocess.run([str(tools[2]), "--notes", str(co)], check=True, capture_output=True,
                                text=True).stdout
    out: dict[str, dict[str, int]] = {}
    name = None
    for line in notes.splitlines():
        m = re.match(r"\s*\.name:\s+(\S+)", line)
        if m:
            name = m.group(1)
            out.setdefault(name, {})
            continue
        m = re.match(r"\s*\.(private_segment_fixed_size|vgpr_count|sgpr_count):\s+(\d+)", line)
        if m and name is not None:
            out[name][m.group(1)] = int(m.group(2))
    return out


def test_no_kernel_spills_to_scratch(tmp_path: Path) -> None:
    kernels = _kernels(tmp_path)
    assert len(kernels) > 100
    hot = [k for k in kernels if re.search(r"k_forward|k_tile|k_finalize|k_update|k_backward|k_merge", k)]
    assert len(hot) > 20
    # every source file's kernels are there (one bundle each)
    for name in ("k_site_eval", "k_merge_index", "k_forward"):
        assert any(name in k for k in kernels), name
    spilling = {k: v["private_segment_fixed_size"] for k, v in kernels.items()
                if v.get("private_segment_fixed_size", 0) > 0 and not ALLOWED.search(k)}
    assert not spilling, f"kernels using scratch: {spilling}"
