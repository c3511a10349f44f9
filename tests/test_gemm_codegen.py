"""Properties of the compiled GEMM kernel that its LDS ring depends on (CPU: hipcc cross-compiles).

The ring's barrier at stage u waits for `vmcnt <=` the slice instructions issued in the
(slots - 2) stages before u (plus, for Q4_K, the one split-sum load issued at a super-block's first
stage): vector memory loads complete in issue order, so every load issued before those has landed.
That holds only if each slice instruction is issued on every path, so no direct-to-LDS load may sit
where an `s_cbranch_execz` can jump over it, and every barrier must use the count of its stage.
"""
from __future__ import annotations

import os
import re
import shutil
import subprocess

import pytest

from apeiron_amd import build

HIPCC = build.HIPCC
KS = 64  # K depth of one stage
TYPES = {8: "Q8_0", 12: "Q4_K", 14: "Q6_K"}


def expected_vmcnt(t: int, waves: int, slots: int) -> list[int]:
    """The count of each of the loop's four stages (u = 0..3 of a super-block)."""
    tok = 64 if t == 12 else 128
    an = tok * KS * 2 // 1024 // waves
    xn = 1 if t == 12 else 0  # Q4_K split sums: one load per wave at a super-block's stage 0
    return [sum(an + (xn if v % 4 == 0 else 0) for v in range(u - (slots - 2), u)) for u in range(4)]


@pytest.fixture(scope="module")
def gemm_asm(tmp_path_factory):
    if not (os.path.exists(HIPCC) or shutil.which(HIPCC)):
        pytest.skip("hipcc not available")
    out = tmp_path_factory.mktemp("asm") / "ah_gemm.s"
    flags = [f for f in build.FLAGS if f not in ("-shared", "-fPIC")]
    cmd = [HIPCC, *flags, "--cuda-device-only", "-S", "-x", "hip",
           os.path.join(build.CSRC, "ah_gemm.hip"), "-o", str(out)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-2000:]
    return out.read_text().split("\n")


def skipped_by_execz(body, i, label):
    """Instructions a forward `s_cbranch_execz label` at body[i] jumps over (none for a backward
    branch: a loop's back edge skips nothing after it)."""
    labels = {l[:-1]: j for j, l in enumerate(body) if l.endswith(":") and not l.startswith(";")}
    tgt = labels.get(label)
    if tgt is None or tgt < i:
        return []
    return body[i + 1:tgt]


def kernels(lines):
    for i, l in enumerate(lines):
        m = re.match(r"^(_ZN12_GLOBAL__N_114gemm_rb_kernelILi(\d+)ELi(\d+)ELi(\d+)E\S*):", l)
        if m:
            end = next(j for j in range(i, len(lines)) if "s_endpgm" in lines[j])
            yield (int(m.group(2)), int(m.group(3)), int(m.group(4))), [x.strip() for x in lines[i:end]]


def test_every_form_is_compiled(gemm_asm):
    forms = {k for k, _ in kernels(gemm_asm)}
    assert {(8, 4, 4), (8, 2, 2), (8, 2, 4), (12, 4, 4), (14, 4, 4), (14, 2, 2), (14, 2, 4)} <= forms


def ring_and_epilogue_barriers(body):
    """The ring's barriers (each behind a vector memory wait) and the others: the exact path's
    LDS-only barriers in the epilogue (its token windows), which must all follow the ring's."""
    bars = [i for i, l in enumerate(body) if l.startswith("s_barrier")]
    ring = [i for i in bars if re.match(r"s_waitcnt vmcnt\(\d+\) lgkmcnt\(0\)$", body[i - 1])]
    rest = [i for i in bars if i not in ring]
    for i in rest:
        assert body[i - 1] == "s_waitcnt lgkmcnt(0)" and (not ring or i > ring[-1]), (i, body[i - 1])
    return ring, rest


def test_ring_barriers_wait_for_the_slice_count(gemm_asm):
    for (t, waves, slots), body in kernels(gemm_asm):
        want = expected_vmcnt(t, waves, slots)
        bars, _ = ring_and_epilogue_barriers(body)
        assert len(bars) == 4, (t, waves, slots, len(bars))  # the loop body's four stages, in order
        for i, w in zip(bars, want):
            m = re.match(r"s_waitcnt vmcnt\((\d+)\) lgkmcnt\(0\)", body[i - 1])
            assert m and int(m.group(1)) == w, (TYPES[t], waves, slots, body[i - 1], want)


def test_mixed_kquant_kernel_barriers(gemm_asm):
    """The grid of Q4_K and Q6_K parts holds both bodies on a 4-slot ring of 4 waves; each
    body's barriers wait for its own stage counts and no slice load sits behind an execz branch."""
    starts = [i for i, l in enumerate(gemm_asm) if re.match(r"^_ZN12_GLOBAL__N_121gemm_rb_kquant_kernel\S*:", l)]
    assert starts
    end = next(j for j in range(starts[0], len(gemm_asm)) if "s_endpgm" in gemm_asm[j])
    body = [x.strip() for x in gemm_asm[starts[0]:end]]
    q4, q6 = expected_vmcnt(12, 4, 4), expected_vmcnt(14, 4, 4)
    seen = []
    for i, l in enumerate(body):
        if l.startswith("s_barrier"):
            m = re.match(r"s_waitcnt vmcnt\((\d+)\) lgkmcnt\(0\)$", body[i - 1])
            if m:
                seen.append(int(m.group(1)))
        m = re.match(r"s_cbranch_execz\s+(\S+)", l)
        if m:
            for x in skipped_by_execz(body, i, m.group(1)):
                assert not (x.startswith("buffer_load") and x.endswith(" lds")), x
    # four stages in each body, in loop order, one body after the other
    assert seen in (q4 + q6, q6 + q4), (seen, q4, q6)


def test_no_slice_load_can_be_skipped(gemm_asm):
    def is_slice(l):
        return l.startswith("buffer_load") and l.endswith(" lds")

    for (t, waves, slots), body in kernels(gemm_asm):
        assert any(is_slice(l) for l in body), (t, waves, slots)
        for i, l in enumerate(body):
            m = re.match(r"s_cbranch_execz\s+(\S+)", l)
            if not m:
                continue
            for x in skipped_by_execz(body, i, m.group(1)):
                assert not is_slice(x), (TYPES[t], waves, slots, i, x)


def test_int8_design_ring(gemm_asm):
    """The int8 kernels (Q8_0 and Q4_K, W waves, 3-slot ring, stages of 4 blocks): each wave
    issues 16/W activation loads and one block-factor load per stage (Q4_K one more, the scaled
    code sums), every ring barrier waits for one stage's slice (the weights of the stage are issued
    before its slice, so they complete too), and no slice load sits behind an execz branch."""
    seen = set()
    for i, l in enumerate(gemm_asm):
        m = re.match(r"^(_ZN12_GLOBAL__N_114gemm_i8_kernelILi(\d+)ELi(\d+)E\S*):", l)
        if not m:
            continue
        t, w = int(m.group(2)), int(m.group(3))
        seen.add((t, w))
        end = next(j for j in range(i, len(gemm_asm)) if "s_endpgm" in gemm_asm[j])
        body = [x.strip() for x in gemm_asm[i:end]]
        want = 16 // w + (2 if t == 12 else 1)
        bars, _ = ring_and_epilogue_barriers(body)
        assert len(bars) == 2, (w, len(bars))  # the loop body runs two stages
        for k in bars:
            mm = re.match(r"s_waitcnt vmcnt\((\d+)\) lgkmcnt\(0\)$", body[k - 1])
            assert mm and int(mm.group(1)) == want, (w, body[k - 1], want)
        slices = [x for x in body if x.startswith("buffer_load") and x.endswith(" lds")]
        assert len(slices) == 4 * want, (w, len(slices))  # prologue 2 stages + 2 in the loop
        for k, x in enumerate(body):
            mm = re.match(r"s_cbranch_execz\s+(\S+)", x)
            if mm:
                for y in skipped_by_execz(body, k, mm.group(1)):
                    assert not (y.startswith("buffer_load") and y.endswith(" lds")), (t, w, y)
    assert seen == {(8, 2), (8, 4), (12, 2), (12, 4)}, seen


@pytest.fixture(scope="module")
def gemv_asm(tmp_path_factory):
    if not (os.path.exists(HIPCC) or shutil.which(HIPCC)):
        pytest.skip("hipcc not available")
    out = tmp_path_factory.mktemp("asm") / "ah_gemv.s"
    flags = [f for f in build.FLAGS if f not in ("-shared", "-fPIC")]
    cmd = [HIPCC, *flags, "--cuda-device-only", "-S", "-x", "hip",
           os.path.join(build.CSRC, "ah_gemv.hip"), "-o", str(out)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-2000:]
    return out.read_text().split("\n")


def test_no_packed_fp32_instructions(gemm_asm, gemv_asm):
    """Every HIP translation unit is built with packed FP32 disabled, and no kernel contains
    v_pk_add_f32 / v_pk_mul_f32 / v_pk_fma_f32 (some of their forms have given wrong results on
    these devices without an error)."""
    i = build.FLAGS.index("-packed-fp32-ops")
    assert build.FLAGS[i - 1] == "-Xclang" and build.FLAGS[i - 2] == "-target-feature"
    for asm in (gemm_asm, gemv_asm):
        bad = [l.strip() for l in asm if re.match(r"\s*v_pk_(add|mul|fma)_f32\b", l)]
        assert not bad, bad[:5]


def test_no_kernel_spills(gemm_asm, gemv_asm):
    """No kernel of either translation unit keeps registers in scratch memory: each kernel's
    `.private_segment_fixed_size` is 0 (a spill would add scratch traffic to every launch)."""
    for asm in (gemm_asm, gemv_asm):
        sizes = [int(m.group(1)) for l in asm if (m := re.match(r"\s*\.private_segment_fixed_size:\s*(\d+)", l))]
        assert len(sizes) >= 10
        assert max(sizes) == 0, [s for s in sizes if s]
