"""Static check of the gfx950 code of the decode kernels: no instruction may touch the
accumulators an inline-asm MFMA writes within the hazard window behind it.

The compiler's hazard recognizer does not look inside inline asm, so a register copy or VALU
op that the compiler places right behind an asm MFMA block (e.g. where two asm paths join)
gets no wait states and can read stale accumulator values.  The asm blocks of the kernels
end their own windows (acc_settle8) where they hand the accumulators to compiled code; this
test compiles the kernel source to device assembly with the build's flags and walks every
path (branches followed) from each asm MFMA for WAIT wait states.

The same assembly is checked for the other blind spot of inline asm: the LDS-DMA loads of
the 32-cell kernel's ring are invisible to the compiler's wait insertion, so a wait it places
in the step loop for a load of its own drains the whole ring every step.  And for register
spills: no kernel may touch scratch memory inside a step loop (the innermost loops that
issue MFMAs); the one kernel with a spill (the q8_0 16-cell kernel at 48 rows, 36 bytes)
keeps it in the piece's set-up and epilogue.
"""
import importlib.util
import pathlib
import re
import subprocess

import pytest

ROOT = pathlib.Path(__file__).resolve().parent.parent
BUILD = ROOT / "sixi-asi_amd" / "build.py"

# v_mfma_f32_16x16x32_f16 is 8 passes: a VALU read of its result needs 11 wait states on
# gfx950 and an overlapping SrcC read by a different-size MFMA up to 19; the window here is
# wider than both.
WAIT = 24

_REG = re.compile(r"\ba\[(\d+)(?::(\d+))?\]|\ba(\d+)\b")


def _agprs(text):
    out = set()
    for m in _REG.finditer(text):
        if m.group(3) is not None:
            out.add(int(m.group(3)))
        else:
            lo = int(m.group(1))
            out.update(range(lo, int(m.group(2) or lo) + 1))
    return out


def _functions(asm):
    for name in re.findall(r"\.type\s+(\S+),@function", asm):
        i = asm.index(name + ":")
        j = asm.find(".Lfunc_end", i)
        yield name, asm[i:j].splitlines()


def _parse(lines):
    labels, ins, in_asm = {}, [], False
    for raw in lines:
        t = raw.strip()
        if "ASMSTART" in t:
            in_asm = True
            continue
        if "ASMEND" in t:
            in_asm = False
            continue
        if t.startswith(";"):
            continue
        t = t.split(";")[0].strip()
        if not t:
            continue
        if t.endswith(":"):
            labels[t[:-1]] = len(ins)
            continue
        if t.startswith("."):
            continue
        ins.append((t, in_asm))
    return labels, ins


def hazards(asm, wait=WAIT):
    """(function, asm MFMA, offending instruction) for every touch of an asm MFMA's result
    registers within `wait` wait states on any path (s_nop N counts N + 1)."""
    found = []
    for name, lines in _functions(asm):
        labels, ins = _parse(lines)
        for k, (t, is_asm) in enumerate(ins):
            if not (is_asm and t.startswith("v_mfma")):
                continue
            dst = _agprs(t.split(",")[0])
            stack, seen = [(k + 1, 0)], set()
            while stack:
                p, w = stack.pop()
                while p < len(ins) and w < wait and (p, w) not in seen:
                    seen.add((p, w))
                    u, u_asm = ins[p]
                    op = u.split()[0]
                    if op.startswith("v_mfma") and u_asm:
                        # a later asm MFMA may accumulate into it (tied SrcC), not read it as A/B
                        srcs = u.split(None, 1)[1].split(",")[1:3]
                        if _agprs(",".join(srcs)) & dst:
                            found.append((name, t, u))
                    elif _agprs(u) & dst:
                        found.append((name, t, u))
                    w += int(u.split()[1], 0) + 1 if op == "s_nop" else 1
                    if op == "s_endpgm":
                        break
                    if op == "s_branch":
                        p = labels[u.split()[1]]
                        continue
                    if op.startswith("s_cbranch"):
                        stack.append((labels[u.split()[1]], w))
                    p += 1
    return found


_TOY = """
\t.type\t_Zk,@function
_Zk:
\t;;#ASMSTART
\ts_nop 2
\tv_mfma_f32_16x16x32_f16 a[0:3], v[0:3], v[4:7], a[0:3]
\t;;#ASMEND
{between}
\tv_accvgpr_read_b32 v8, a2
\ts_endpgm
.Lfunc_end0:
"""


def test_checker_finds_a_planted_hazard():
    assert len(hazards(_TOY.format(between=""))) == 1
    # a branch to a block that reads the result is followed
    branchy = _TOY.format(between="\ts_cbranch_scc1 .LBB0_2\n\ts_nop 7\n\ts_nop 7\n\ts_nop 7\n"
                                   "\ts_endpgm\n.LBB0_2:")
    assert len(hazards(branchy)) == 1
    # other registers, and reads past the window, are fine
    assert hazards(_TOY.format(between="").replace("a2", "a4")) == []
    assert hazards(_TOY.format(between="\ts_nop 7\n\ts_nop 7\n\ts_nop 7")) == []


@pytest.fixture(scope="module")
def decode_asm(tmp_path_factory):
    """gfx950 assembly of fa_decode.hip, built with the library's flags."""
    spec = importlib.util.spec_from_file_location("sixi_build", BUILD)
    build = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(build)
    try:
        hipcc = build._hipcc()
    except RuntimeError:
        pytest.skip("hipcc not available")
    flags = [f for f in build.flags_for("fa_decode.hip") if f != "-fPIC"]
    out = tmp_path_factory.mktemp("asm") / "fa_decode.s"
    proc = subprocess.run([hipcc, *flags, "--cuda-device-only", "-S", "-o", str(out), str(build.CSRC / "fa_decode.hip")],
                          stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    assert proc.returncode == 0, proc.stdout[-2000:]
    return out.read_text()


def test_decode_kernels_have_no_asm_mfma_hazards(decode_asm):
    assert decode_asm.count("v_mfma_f32_16x16x32_f16 a[") > 0, "no asm MFMAs found: the check would be vacuous"
    bad = hazards(decode_asm)
    assert not bad, f"{len(bad)} hazards, first: {bad[:3]}"


def drains_before_lds_reads(asm, kernel_pattern):
    """Compiler-placed vmcnt waits right before an LDS read, per kernel matching the pattern.
    In the 32-cell kernel every vector-memory load of the step loop is an LDS-DMA load issued by
    inline asm, which the compiler does not see; a wait it places before an LDS read stands for
    a load it believes pending (from before the loop) and, executed in the loop, drains the DMA
    ring every step."""
    out = {}
    for name, lines in _functions(asm):
        if not re.search(kernel_pattern, name):
            continue
        body = [l.strip() for l in lines]
        n = sum(1 for k in range(1, len(body) - 1)
                if re.match(r"s_waitcnt\b.*vmcnt", body[k]) and "ASMSTART" not in body[k - 1]
                and body[k + 1].startswith("ds_read"))
        out[name] = n
    return out


def test_wide_decode_step_loops_do_not_drain_the_dma_ring(decode_asm):
    # fast (mode 0) and staged-mask (mode 2) variants of decode_wide<NTW, RS, MODE, D>
    found = drains_before_lds_reads(decode_asm, r"decode_wideILi\d+ELi\d+ELi[02]ELi\d+E")
    assert len(found) >= 8, found
    bad = {k: v for k, v in found.items() if v}
    assert not bad, bad


def scratch_in_step_loops(asm):
    """(function, instruction) for every scratch access inside a step loop: a loop (label ..
    backward branch) that issues MFMAs and contains no smaller loop that does."""
    found = []
    for name, lines in _functions(asm):
        labels, ins = _parse(lines)
        ops = [t for t, _ in ins]
        loops = []
        for k, t in enumerate(ops):
            parts = t.split()
            if (parts[0].startswith("s_cbranch") or parts[0] == "s_branch") and len(parts) > 1:
                a = labels.get(parts[1])
                if a is not None and a < k and any(u.startswith("v_mfma") for u in ops[a:k + 1]):
                    loops.append((a, k))
        steps = [(a, b) for a, b in loops
                 if not any((c, d) != (a, b) and a <= c and d <= b for c, d in loops)]
        for a, b in steps:
            found += [(name, u) for u in ops[a:b + 1] if u.startswith("scratch_")]
    return found


def test_checker_finds_scratch_in_a_step_loop():
    toy = ("\t.type\t_Zk,@function\n_Zk:\n.LBB0_1:\n\tv_mfma_f32_16x16x32_f16 v[0:3], v[4:7], v[8:11], v[0:3]\n"
           "\t{mid}\n\ts_cbranch_scc1 .LBB0_1\n\tscratch_load_dword v1, off, off\n\ts_endpgm\n.Lfunc_end0:\n")
    assert len(scratch_in_step_loops(toy.format(mid="scratch_store_dword off, v1, off"))) == 1
    assert scratch_in_step_loops(toy.format(mid="v_mov_b32 v1, v2")) == []


def test_decode_kernels_call_no_functions(decode_asm):
    # every piece function is inlined into its kernel (an out-of-line one gave wrong results);
    # s_setpc_b64 alone is the compiler's far branch, s_swappc a call
    assert "s_swappc" not in decode_asm
    names = re.findall(r"\.type\s+(\S+),@function", decode_asm)
    assert names and all(re.search(r"sixi.*(decode_|merge)", n) for n in names), names[:5]


def test_decode_kernels_touch_no_scratch_in_step_loops(decode_asm):
    bad = scratch_in_step_loops(decode_asm)
    assert not bad, f"{len(bad)} scratch accesses in step loops, first: {bad[:3]}"


def _asm_of(src, tmp_path_factory):
    """gfx950 assembly of one HIP source of the library, built with the library's flags."""
    spec = importlib.util.spec_from_file_location("sixi_build", BUILD)
    build = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(build)
    try:
        hipcc = build._hipcc()
    except RuntimeError:
        pytest.skip("hipcc not available")
    flags = [f for f in build.flags_for(src) if f != "-fPIC"]
    out = tmp_path_factory.mktemp("asm") / (src + ".s")
    proc = subprocess.run([hipcc, *flags, "--cuda-device-only", "-S", "-o", str(out), str(build.CSRC / src)],
                          stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    assert proc.returncode == 0, proc.stdout[-2000:]
    return out.read_text()


def kernels_with_scratch(asm):
    """(kernel, bytes) for every kernel whose metadata reserves private (scratch) memory."""
    meta = asm[asm.index("amdhsa.kernels:"):]
    found = []
    for blk in meta.split("\n  - ")[1:]:
        # kernel-level keys are indented four spaces (argument keys eight)
        name = re.search(r"^    \.name:\s+(\S+)", blk, re.M)
        size = re.search(r"^    \.private_segment_fixed_size:\s+(\d+)", blk, re.M)
        if name and size and int(size.group(1)) > 0:
            found.append((name.group(1), int(size.group(1))))
    return found


def test_scratch_checker_reads_kernel_metadata():
    meta = ("amdhsa.kernels:\n  - .agpr_count: 0\n    .args:\n      - .name: a\n        .offset: 0\n"
            "    .name: k_a\n    .private_segment_fixed_size: 0\n"
            "  - .agpr_count: 0\n    .name: k_b\n    .private_segment_fixed_size: 36\n")
    assert kernels_with_scratch(meta) == [("k_b", 36)]


@pytest.fixture(scope="module")
def prefill_asm(tmp_path_factory):
    return _asm_of("fa_prefill.hip", tmp_path_factory)


def test_prefill_kernels_touch_no_scratch_in_tile_loops(prefill_asm):
    assert prefill_asm.count("v_mfma") > 0
    bad = scratch_in_step_loops(prefill_asm)
    assert not bad, f"{len(bad)} scratch accesses in tile loops, first: {bad[:3]}"


def test_attention_kernels_use_no_scratch(decode_asm, prefill_asm):
    # every decode, merge and prefill variant the library can launch keeps all its values in
    # registers and LDS (no spill anywhere, prologue and epilogue included)
    for asm in (decode_asm, prefill_asm):
        assert asm.count(".private_segment_fixed_size:") > 5
        bad = kernels_with_scratch(asm)
        assert not bad, f"{len(bad)} kernels with scratch: {bad[:4]}"


@pytest.mark.parametrize("src", ["fa_q8_stage.hip", "kv_write.hip", "layer_prologue.hip", "gdn_verify.hip"])
def test_other_kernels_use_no_scratch(src, tmp_path_factory):
    asm = _asm_of(src, tmp_path_factory)
    assert asm.count(".private_segment_fixed_size:") > 0
    bad = kernels_with_scratch(asm)
    assert not bad, f"{len(bad)} kernels with scratch: {bad[:4]}"


def kernel_vgprs(asm, fragment):
    """{kernel: VGPRs + AGPRs} from the metadata of every kernel whose name contains fragment."""
    meta = asm[asm.index("amdhsa.kernels:"):]
    found = {}
    for blk in meta.split("\n  - ")[1:]:
        name = re.search(r"^    \.name:\s+(\S+)", blk, re.M)
        vgpr = re.search(r"^    \.vgpr_count:\s+(\d+)", blk, re.M)
        if name and vgpr and fragment in name.group(1):
            found[name.group(1)] = int(vgpr.group(1))
    return found


def test_gdn_chunked_kernel_fits_four_work_groups_per_cu(tmp_path_factory):
    # The chunked GDN kernel runs four 4-wave work-groups per CU (four waves per SIMD) only at
    # <= 128 registers; at 129 it drops to three and the 32 x 16 verify batch slows by ~5 %, with
    # every output unchanged, so only this test would notice.
    counts = kernel_vgprs(_asm_of("gdn_verify.hip", tmp_path_factory), "gdn_verify_chunked_kernel")
    assert len(counts) == 4, counts
    assert max(counts.values()) <= 128, counts
