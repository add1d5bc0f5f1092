"""Code-generation checks of the prefill kernel (CPU only: hipcc -S for gfx950).

The tile loop copies K/V tiles into LDS with global_load_lds instructions that
the compiler does not see.  A compiler-inserted full ``s_waitcnt vmcnt(0)``
between the pair barrier and the first matrix product would also wait for the
copies issued right after the barrier, so each pair of tiles would wait for
the next pair to land.  This checks, for the page-per-tile kernels (block
sizes that are multiples of 64, the common case), that the only full
vector-memory wait before the first MFMA after a barrier is the barrier's own.
"""

import re
import subprocess

import pytest

from mini_engine_hip import build as hip_build

SOURCE = hip_build.SOURCE_DIR / "paged_prefill.hip"


@pytest.fixture(scope="module")
def prefill_asm(tmp_path_factory):
    try:
        hipcc = hip_build._hipcc()
    except RuntimeError as exc:
        pytest.skip(str(exc))
    out = tmp_path_factory.mktemp("asm") / "paged_prefill.s"
    cmd = [hipcc, *hip_build.HIP_FLAGS, f"-I{hip_build.INCLUDE_DIR}", "--cuda-device-only", "-S",
           str(SOURCE), "-o", str(out)]
    result = subprocess.run(cmd, capture_output=True, text=True)
    assert result.returncode == 0, result.stderr[-2000:]
    return out.read_text()


def kernels(asm):
    """(name, instructions) of each MFMA prefill kernel, comments and directives dropped."""
    found = []
    for body in re.split(r"\n(?=_ZN\S*:)", asm):
        m = re.match(r"(_ZN\S*paged_prefill_mfma_kernel\S*):", body)
        if m:
            ins = [l.strip() for l in body.split("\n") if l.strip() and not l.strip().startswith((";", "."))]
            found.append((m.group(1), ins))
    return found


def stray_waits(ins):
    """Full vmcnt waits between a barrier and the first MFMA after it, other
    than the wait that directly precedes a barrier, issued while tile copies
    (global_load_lds) are in flight -- a full wait with no copy outstanding
    (e.g. for an item's metadata before its first copy) delays nothing."""
    stray, armed, pending, copies = [], False, None, False
    for i, s in enumerate(ins):
        if s.startswith("global_load_lds"):
            copies = True
        if s.startswith("s_endpgm"):
            # Execution does not fall through: the instructions laid out
            # next belong to blocks reached by branches from elsewhere.
            armed, pending = False, None
        elif s.startswith("s_barrier"):
            armed, pending = True, None
        elif s.startswith("s_waitcnt") and "vmcnt(0)" in s:
            if armed and copies and not (i + 1 < len(ins) and ins[i + 1].startswith("s_barrier")):
                pending = (i, s)
            copies = False
        elif armed and s.startswith("v_mfma"):
            if pending:
                stray.append(pending)
            armed, pending = False, None
    return stray


def test_page_per_tile_kernels_do_not_wait_for_inflight_copies(prefill_asm):
    tile_kernels = [(n, ins) for n, ins in kernels(prefill_asm) if "ELi2E" in n]
    assert len(tile_kernels) == 32  # fp16/bf16 x walk/no walk x tile shape 128/256 x full/zero-padded rows x paged/dense
    for name, ins in tile_kernels:
        assert sum(s.startswith("v_mfma") for s in ins) > 0, name
        assert stray_waits(ins) == [], name


def test_stray_wait_detector_flags_a_planted_wait():
    """The detector itself: a full wait between the barrier and the first
    product is reported; the barrier's own wait is not."""
    clean = ["s_waitcnt vmcnt(0) lgkmcnt(0)", "s_barrier", "global_load_lds_dwordx4 v0, off",
             "s_waitcnt lgkmcnt(3)", "v_mfma_f32_16x16x32_bf16 v[0:3], v[4:7], v[8:11], 0"]
    assert stray_waits(clean) == []
    planted = clean[:3] + ["s_waitcnt vmcnt(0) lgkmcnt(3)"] + clean[4:]
    assert stray_waits(planted) == [(3, "s_waitcnt vmcnt(0) lgkmcnt(3)")]
    # A full wait before any copy of the barrier's interval is issued is harmless.
    early = clean[:2] + ["s_waitcnt vmcnt(0)"] + clean[2:]
    assert stray_waits(early) == []
    # So is the drain before a work-group ends: the product laid out after
    # s_endpgm is not executed next.
    ending = clean[:3] + ["s_waitcnt vmcnt(0)", "s_endpgm"] + clean[4:]
    assert stray_waits(ending) == []
