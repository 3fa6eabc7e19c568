"""The shape of the built gfx950 code object (amd.c_amd/amdc_kernels.hsaco).

A CPU test: it disassembles the code object this repository builds (llvm-objdump
of our own AMD code, the counterpart of the reference's tools/check_objdump.sh:1-25,
which asserts dot4 counts, b128 loads and no scratch on its RDNA4 build) and checks
what the kernels rely on but the compiler cannot see:

* no kernel uses scratch memory or spills vector registers (SGPR spills go
  to VGPR lanes, not memory: amdc_chain has a few);
* no packed FP32 instruction (v_pk_add/mul/fma_f32) is emitted anywhere;
* the integer block dots run on v_dot4_i32_i8 in the decode kernels, and the
  verify and prefill kernels run on MFMA;
* every buffer load into the LDS has at least one instruction between the
  write of m0 that addresses it and the load (the gfx9 hazard); in the verify
  kernels whose LDS loads are inline asm (lds_load16), m0 is written only right
  before such a load;
* the explicit waits of those kernels and of the Q6_K verify kernels (vm_wait,
  marked by expcnt(6)): a plane's
  ring slot was filled by a load into the LDS issued one ring step earlier,
  and the count n of the wait must leave that load complete, i.e. at least n
  vector memory instructions were issued after it. The check walks the
  compiled instruction order, on the first pass through the tile loop (after
  the prologue) and in the steady state (after the previous iteration).
"""
import os
import re
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HSACO = os.path.join(ROOT, "amd.c_amd", "amdc_kernels.hsaco")
LLVM = "/opt/rocm/llvm/bin"

# kernels whose loads into the LDS are inline asm, with (ring steps, LDS loads per ring step, explicit
# waits per tile): gemv8_body<KIND, NS, NH, WS>: NS steps, SC * (2 if WS == 1 else 1) loads per step,
# a wait per plane
INLINE_LDS = {
    "amdc_gemv_q4_0_v8": (2, 1, 8),
    "amdc_gemv_q4_k_v8": (2, 1, 8),
    "amdc_gemv_q8_0_v8": (2, 4, 8),
    "amdc_gemv_q4_0_v16": (2, 1, 8),
    "amdc_gemv_q4_k_v16": (2, 1, 8),
    "amdc_gemv_q8_0_v16": (1, 4, 8),
}
# kernels whose loads into the LDS are the compiler's builtin but whose ring reads wait explicitly:
# gemv8_q6k_body<NQ, NS>: NS steps of 6 loads, a wait per step (4 per tile)
BUILTIN_LDS = {
    "amdc_gemv_q6_k_v8": (2, 6, 4),
    "amdc_gemv_q6_k_v16": (1, 6, 4),
}


def _tool(name):
    p = os.path.join(LLVM, name)
    return p if os.path.exists(p) else shutil.which(name)


@pytest.fixture(scope="module")
def code(tmp_path_factory):
    if not os.path.exists(HSACO):
        pytest.skip("amdc_kernels.hsaco is not built")
    bundler, objdump, readelf = _tool("clang-offload-bundler"), _tool("llvm-objdump"), _tool("llvm-readelf")
    if not (bundler and objdump and readelf):
        pytest.skip("the ROCm LLVM tools are not installed")
    co = str(tmp_path_factory.mktemp("isa") / "k.co")
    subprocess.run([bundler, "--unbundle", "--type=o", f"--input={HSACO}", "--targets=hipv4-amdgcn-amd-amdhsa--gfx950",
                    f"--output={co}"], check=True)
    dis = subprocess.run([objdump, "-d", "--mcpu=gfx950", co], check=True, capture_output=True, text=True).stdout
    notes = subprocess.run([readelf, "--notes", co], check=True, capture_output=True, text=True).stdout
    funcs, cur = {}, None
    for line in dis.splitlines():
        m = re.match(r"^([0-9a-f]+) <(\w+)>:", line)
        if m:
            cur = funcs.setdefault(m.group(2), [])
            continue
        m = re.match(r"^\s+(\w+)\s*([^/]*?)\s*//\s*([0-9A-F]+):", line)
        if m and cur is not None:
            cur.append((int(m.group(3), 16), m.group(1), m.group(2)))
    meta = {}
    for block in re.split(r"\n\s+- \.", notes):
        name = re.search(r"\.name:\s+(\w+)", block)
        if name and name.group(1).startswith("amdc_"):
            fields = dict(re.findall(r"\.(\w+):\s+(\d+)\s*$", block, re.M))
            meta[name.group(1)] = {k: int(v) for k, v in fields.items()}
    return funcs, meta


def is_vmem(mn):
    return mn.startswith(("buffer_", "global_", "flat_", "scratch_"))


def is_lds_dma(mn, ops):
    return mn.startswith("buffer_load") and re.search(r"\blds\b", ops) is not None


def writes_m0(mn, ops):
    return mn.startswith("s_") and re.match(r"m0\b", ops) is not None


def test_kernels_present(code):
    funcs, meta = code
    kernels = [k for k in funcs if k.startswith("amdc_")]
    assert len(kernels) >= 50
    assert set(kernels) <= set(meta), "every kernel has metadata"


def test_no_scratch_no_spills(code):
    _, meta = code
    bad = {k: v for k, v in meta.items()
           if v.get("private_segment_fixed_size", 0) or v.get("vgpr_spill_count", 0)}
    assert not bad, f"kernels using scratch or spilling: {sorted(bad)}"


def test_no_packed_fp32(code):
    funcs, _ = code
    hits = [(k, mn) for k, ins in funcs.items() for _, mn, _ in ins if re.match(r"v_pk_(add|mul|fma)_f32", mn)]
    assert not hits, hits[:5]


def test_decode_dots_on_dot4(code):
    funcs, _ = code
    dec = [k for k in funcs if re.match(r"amdc_gemv_q(4_0|4_k|8_0|6_k)_(s\d|s1w|xs\d|xw\d|n\d|p1|p2|pn|x1|m1)$", k)]
    assert len(dec) >= 16
    for k in dec:
        n = sum(re.match(r"v_dot4c?_i32_i8", mn) is not None for _, mn, _ in funcs[k])
        assert n >= 8, f"{k}: {n} v_dot4_i32_i8"


def test_verify_and_gemm_on_mfma(code):
    funcs, _ = code
    mm = [k for k in funcs if re.match(r"amdc_(gemv_\w+_v(8|16)|gemmh_\w+|gemm_q\w+)$", k)]
    assert len(mm) >= 16
    for k in mm:
        assert any(mn.startswith("v_mfma_") for _, mn, _ in funcs[k]), k


def test_m0_hazard(code):
    """No buffer load into the LDS directly after the write of m0 it reads."""
    funcs, _ = code
    n = 0
    for k, ins in funcs.items():
        for i, (_, mn, ops) in enumerate(ins):
            if is_lds_dma(mn, ops):
                n += 1
                assert i > 0 and not writes_m0(*ins[i - 1][1:]), f"{k} at {ins[i][0]:#x}: m0 written right before the load"
    assert n > 0


def test_inline_lds_m0_only_for_the_load(code):
    """In the lds_load16 kernels m0 is set only as `s_mov_b32 m0; s_nop 0; buffer_load ... lds`."""
    funcs, _ = code
    for k in INLINE_LDS:
        ins = funcs[k]
        loads = 0
        for i, (_, mn, ops) in enumerate(ins):
            if writes_m0(mn, ops):
                assert mn == "s_mov_b32" and ins[i + 1][1] == "s_nop" and is_lds_dma(*ins[i + 2][1:]), f"{k} at {ins[i][0]:#x}"
            if is_lds_dma(mn, ops):
                loads += 1
                assert writes_m0(*ins[i - 2][1:]), f"{k} at {ins[i][0]:#x}: the load is not paired with its m0 write"
        assert loads >= 8, k


def _check_waits(name, seq, marks, ns, dps):
    """seq: instructions in issue order; marks: indices of the waits to check."""
    for j in marks:
        _, _, ops = seq[j]
        m = re.search(r"vmcnt\((\d+)\)", ops)
        n = int(m.group(1)) if m else 63
        lds = [i for i in range(j) if is_lds_dma(seq[i][1], seq[i][2])]
        back = (ns - 1) * dps + 1  # the slot's last load: this many LDS loads back
        assert len(lds) >= back, f"{name} at {seq[j][0]:#x}: no load fills the plane's slot"
        last = lds[-back]
        after = sum(is_vmem(mn) for _, mn, _ in seq[last + 1:j])
        assert after >= n, (f"{name}: the wait at {seq[j][0]:#x} (vmcnt({n})) leaves the LDS load at {seq[last][0]:#x} "
                            f"in flight ({after} vector memory instructions after it)")


def test_explicit_waits_cover_the_ring(code):
    funcs, _ = code
    for k, (ns, dps, nw) in {**INLINE_LDS, **BUILTIN_LDS}.items():
        ins = funcs[k]
        marked = [i for i, (_, mn, ops) in enumerate(ins) if mn == "s_waitcnt" and "expcnt(6)" in ops]
        assert len(marked) == nw, f"{k}: {len(marked)} marked waits ({nw} per tile expected)"
        # the tile loop: the backward branch whose range holds the marked waits
        loops = [(_target(ins, i), i) for i, (_, mn, _) in enumerate(ins) if mn.startswith(("s_branch", "s_cbranch"))]
        loops = [(s, e) for s, e in loops if s is not None and s <= marked[0] and marked[-1] < e]
        assert loops, f"{k}: no loop around the planes"
        s, e = max(loops, key=lambda x: x[0])
        body = ins[s:e + 1]
        # first pass: the prologue, then the body
        _check_waits(k, ins[:e + 1], marked, ns, dps)
        # steady state: the body after the body
        two = body + body
        _check_waits(k, two, [len(body) + (i - s) for i in marked], ns, dps)


def _target(ins, i):
    """Index of the target of branch i (the operand is a signed word offset from the next instruction)."""
    addr, _, ops = ins[i]
    try:
        off = int(ops.split()[0], 0)
    except (ValueError, IndexError):
        return None
    if off >= 0x8000:
        off -= 0x10000
    t = addr + 4 + 4 * off
    for j, x in enumerate(ins):
        if x[0] == t:
            return j
    return None
