"""The MFMA kernels' instruction schedule, read from the gfx950 assembly (CPU).

The K-split and tile-resident GEMM kernels issue their MFMAs as inline-asm
blocks that accumulate in place (csrc/mfma.h), so their hazard spacing is
written by hand (the compiler's hazard recognizer does not see into the asm).
On gfx950 these patterns gave wrong sums with no error: a VALU instruction
writing a register that an MFMA issued a few instructions earlier still reads
(A, B or C operand), and an independent MFMA writing such a register.  This
test compiles those kernels' sources with the library's own flags (device
code only, to assembly), walks each such kernel's instruction stream with a
window of the last 8 issue slots (an `s_nop n` counts n + 1), and requires
none of those writes in any window.  (Kernels that call the MFMA builtins,
such as attention and the prefill GEMMs, are spaced by the compiler and not
checked here.)  It needs hipcc, not a GPU.
"""

from __future__ import annotations

import re
import shutil
import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT / "maple-flash-dgx-spark_amd"))
import build as libbuild  # noqa: E402

SOURCES = ["dense_mfma.hip", "grouped.hip"]
# kernels whose MFMAs are the inline-asm blocks
HAND_SCHEDULED = re.compile(r"k_tgemm_ks|k_tgemm_xpk|k_rtn4_mfma|k_grouped_(swiglu|down)_(er|ks)")
WINDOW = 8


def _regs(operand: str) -> set[int]:
    operand = operand.strip()
    m = re.match(r"v\[(\d+):(\d+)\]", operand)
    if m:
        return set(range(int(m.group(1)), int(m.group(2)) + 1))
    m = re.match(r"v(\d+)$", operand)
    return {int(m.group(1))} if m else set()


def scan(asm: str) -> dict[str, dict[str, int]]:
    """Per kernel: MFMA count and the number of hazardous writes found."""
    res: dict[str, dict[str, int]] = {}
    name, hist = None, []
    for line in asm.splitlines():
        m = re.match(r"^(_Z\S+):", line)
        if m:
            name, hist = m.group(1), []
            res[name] = {"mfma": 0, "valu_on_operand": 0, "mfma_on_operand": 0}
            continue
        t = line.strip()
        if name is None or not t or t[0] in ";." or t.endswith(":"):
            continue
        parts = t.split(None, 1)
        op = parts[0]
        ops = [o.strip() for o in parts[1].split(",")] if len(parts) > 1 else []
        if op == "s_nop":
            hist.extend([("o", set(), set())] * (int(ops[0], 0) + 1))
            continue
        recent = hist[-WINDOW:]
        if op.startswith("v_mfma"):
            d, a, b, c = (_regs(o) for o in ops[:4])
            res[name]["mfma"] += 1
            for kind, reads, dst in recent:
                # an MFMA that reads the earlier one's result runs after it
                if kind == "m" and d & reads and not ((a | b | c) & dst):
                    res[name]["mfma_on_operand"] += 1
            hist.append(("m", a | b | c, d))
            continue
        writes = op.startswith(("v_", "global_load", "ds_read", "buffer_load")) and not op.startswith(
            ("v_cmp", "v_cmpx"))
        dst = _regs(ops[0]) if writes and ops else set()
        for kind, reads, _ in recent:
            if kind == "m" and dst & reads:
                res[name]["valu_on_operand"] += 1
        hist.append(("o", set(), set()))
    return res


@pytest.mark.skipif(not (Path(libbuild.HIPCC).exists() or shutil.which("hipcc")), reason="hipcc not found")
@pytest.mark.parametrize("src", SOURCES)
def test_no_register_writes_under_inflight_mfma(src, tmp_path):
    out = tmp_path / (src + ".s")
    flags = [f for f in libbuild.FLAGS if f != "-fPIC"]
    cmd = [libbuild.HIPCC, *flags, "--cuda-device-only", "-S", str(libbuild.CSRC / src), "-o", str(out)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    assert res.returncode == 0, res.stderr[-2000:]
    kernels = {k: v for k, v in scan(out.read_text()).items() if v["mfma"] and HAND_SCHEDULED.search(k)}
    assert kernels, f"no hand-scheduled MFMA kernels found in {src}"
    bad = {k[:60]: v for k, v in kernels.items() if v["valu_on_operand"] or v["mfma_on_operand"]}
    assert not bad, bad


def test_scan_flags_a_planted_hazard():
    """The scanner itself: a VALU write to an in-flight MFMA's B operand and an
    independent MFMA writing another's C operand are both counted; the same
    stream with enough wait states between them is clean."""
    planted = """_Zplanted:
	v_mfma_f32_16x16x32_bf16 v[0:3], v[4:7], v[8:11], v[0:3]
	v_mov_b32_e32 v9, 0
	v_mfma_f32_16x16x32_bf16 v[0:3], v[12:15], v[16:19], v[20:23]
"""
    r = scan(planted)["_Zplanted"]
    assert r["mfma"] == 2 and r["valu_on_operand"] == 1 and r["mfma_on_operand"] == 1
    clean = planted.replace("\tv_mov_b32_e32 v9, 0\n", "\ts_nop 7\n\tv_mov_b32_e32 v9, 0\n").replace(
        "\tv_mfma_f32_16x16x32_bf16 v[0:3], v[12:15]", "\ts_nop 7\n\tv_mfma_f32_16x16x32_bf16 v[0:3], v[12:15]")
    r = scan(clean)["_Zplanted"]
    assert r["valu_on_operand"] == 0 and r["mfma_on_operand"] == 0
