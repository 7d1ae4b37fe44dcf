"""Static check of the generated gfx950 code (CPU only: hipcc cross-compiles).

Some MFMAs and the LDS-direct gathers are issued through inline asm (dsa_common.h,
dsa_kvtile.h); the compiler's hazard recognizer does not see inside asm, so those forms carry
their own wait states.  This test compiles the kernels and checks the generated code for the
hazards they must cover, so a compiler or code change that breaks the contract cannot slip
through:
  - no VALU instruction writes a source register of an MFMA in the 2 issue slots before it;
  - an LDS DMA (global_load_lds_*) issues at least 1 wait state after the last M0 write;
  - a vector memory instruction reading an SGPR base issues at least 5 wait states after a
    VALU write (v_readlane / v_readfirstlane) of that SGPR;
  - no instruction other than an MFMA accumulating into the same registers reads an MFMA
    result within 8 (16x16x32) / 12 (32x32x16) wait states (VALU, v_accvgpr_read, store or LDS
    write data).
The distances are what the compiler itself inserts for the same sequences.
"""
import os
import re
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "mcore-bridge_amd", "csrc")
FLAGS = ["--offload-arch=gfx950", "-O3", "-std=c++17", "-Xclang", "-target-feature", "-Xclang",
         "-packed-fp32-ops", "-w", "-S", "--cuda-device-only"]
HAZARD_SLOTS = 2

pytestmark = pytest.mark.skipif(shutil.which("hipcc") is None and not os.path.exists("/opt/rocm/bin/hipcc"),
                                reason="hipcc not available")


def _regs(tok):
    """Register set of an operand token: ('v', i) / ('a', i) entries."""
    m = re.fullmatch(r"([va])\[(\d+):(\d+)\]", tok)
    if m:
        return {(m.group(1), i) for i in range(int(m.group(2)), int(m.group(3)) + 1)}
    m = re.fullmatch(r"([va])(\d+)", tok)
    if m:
        return {(m.group(1), int(m.group(2)))}
    return set()


def _operands(line):
    body = line.split(";")[0].strip()
    parts = body.split(None, 1)
    if len(parts) < 2:
        return parts[0] if parts else "", []
    return parts[0], [t.strip() for t in parts[1].split(",")]


def _sregs(tok):
    m = re.fullmatch(r"s\[(\d+):(\d+)\]", tok)
    if m:
        return {i for i in range(int(m.group(1)), int(m.group(2)) + 1)}
    m = re.fullmatch(r"s(\d+)", tok)
    return {int(m.group(1))} if m else set()


def _mem_violations(asm_text):
    """M0 -> LDS DMA (1 wait state) and VALU SGPR write -> VMEM SGPR read (5 wait states)."""
    bad = []
    since_m0 = 99            # wait states since the last M0 write
    since_sgpr = {}          # SGPR -> wait states since a VALU wrote it
    func = "?"
    for raw in asm_text.split("\n"):
        line = raw.strip()
        m = re.match(r"^(_Z\w+):", line)
        if m:
            func, since_m0, since_sgpr = m.group(1), 99, {}
        if not line or line.startswith((";", ".", "_")) or line.endswith(":"):
            continue
        mn, ops = _operands(line)
        if not mn or not re.match(r"[vsdgb]", mn):
            continue
        if mn.startswith("global_load_lds") and since_m0 < 1:
            bad.append(f"{func}: `{line}` issues {since_m0} wait states after an M0 write")
        if mn.startswith(("global_", "buffer_", "scratch_")):
            for r in set().union(*[_sregs(o) for o in ops]) if ops else set():
                if since_sgpr.get(r, 99) < 5:
                    bad.append(f"{func}: `{line}` reads s{r} {since_sgpr[r]} wait states after a VALU write")
        n = int(ops[0], 0) + 1 if mn == "s_nop" and ops else 1
        since_m0 += n
        for r in since_sgpr:
            since_sgpr[r] += n
        if ops and ops[0] == "m0":
            since_m0 = 0
        if mn.startswith("v_readlane") or mn.startswith("v_readfirstlane"):
            for r in _sregs(ops[0]):
                since_sgpr[r] = 0
    return bad


def _mfma_result_wait(mn):
    return 8 if "16x16" in mn else 12


def _result_violations(asm_text):
    """An MFMA result read by a non-MFMA instruction before the result latency has passed."""
    bad = []
    pending = []   # [wait states since issue, required, dst regs, mnemonic]
    func = "?"
    for raw in asm_text.split("\n"):
        line = raw.strip()
        m = re.match(r"^(_Z\w+):", line)
        if m:
            func, pending = m.group(1), []
        if not line or line.startswith((";", ".", "_")) or line.endswith(":"):
            continue
        mn, ops = _operands(line)
        if not mn or not re.match(r"[vsdgb]", mn):
            continue
        if mn.startswith("v_mfma"):
            srcs = set()
            for t in ops[1:3]:
                srcs |= _regs(t)
            for p in pending:   # A / B operands of a later MFMA are reads too
                if p[0] < p[1] and p[2] & srcs:
                    bad.append(f"{func}: `{line}` reads the result of `{p[3]}` {p[0]} wait states after it")
        else:
            if mn.startswith(("ds_write", "global_store", "buffer_store", "scratch_store", "flat_store")):
                srcs = set().union(*[_regs(t) for t in ops]) if ops else set()
            elif mn.startswith(("v_", "ds_", "global_", "buffer_", "scratch_", "flat_")):
                srcs = set().union(*[_regs(t) for t in ops[1:]]) if len(ops) > 1 else set()
            else:
                srcs = set()
            for p in pending:
                if p[0] < p[1] and p[2] & srcs:
                    bad.append(f"{func}: `{line}` reads the result of `{p[3]}` {p[0]} wait states after it")
        n = int(ops[0], 0) + 1 if mn == "s_nop" and ops else 1
        for p in pending:
            p[0] += n
        pending = [p for p in pending if p[0] < p[1]]
        if mn.startswith("v_mfma"):
            pending.append([0, _mfma_result_wait(mn), _regs(ops[0]), line])
    return bad


def _violations(asm_text):
    bad = []
    window = []   # (slots, mnemonic, written regs) of the last instructions
    func = "?"
    for raw in asm_text.split("\n"):
        line = raw.strip()
        m = re.match(r"^(_Z\w+):", line)
        if m:
            func = m.group(1)
        if not line or line.startswith((";", ".", "_")) or line.endswith(":"):
            continue   # labels keep the window: the fall-through path is checked across them
        mn, ops = _operands(line)
        if not mn or not re.match(r"[vsdgb]", mn):
            continue
        if mn.startswith("v_mfma"):
            srcs = set()
            for t in ops[1:4]:
                srcs |= _regs(t)
            slots = 0
            for s, pmn, wr in reversed(window):
                if slots >= HAZARD_SLOTS:
                    break
                if wr & srcs and not pmn.startswith(("v_mfma", "ds_", "global_", "buffer_")):
                    bad.append(f"{func}: {pmn} writes a source of `{line}`")
                slots += s
            window.append((1, mn, set()))
        else:
            slots = 1
            if mn == "s_nop" and ops:
                slots = int(ops[0], 0) + 1
            written = _regs(ops[0]) if mn.startswith("v_") and ops else set()
            window.append((slots, mn, written))
        window = window[-8:]
    return bad


@pytest.mark.parametrize("src", ["dsa_sparse_fwd.hip", "dsa_sparse_bwd.hip", "dsa_indexer.hip", "dsa_indexer_bwd.hip",
                                 "dsa_dense_kl.hip"])
def test_no_valu_write_right_before_mfma(src, tmp_path):
    out = tmp_path / (src + ".s")
    hipcc = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    subprocess.run([hipcc, *FLAGS, "-o", str(out), os.path.join(CSRC, src)], check=True, cwd=CSRC,
                   capture_output=True, timeout=600)
    text = out.read_text()
    assert "v_mfma" in text
    bad = _violations(text) + _mem_violations(text) + _result_violations(text)
    assert not bad, "\n".join(bad[:20])


def test_checker_flags_a_planted_hazard():
    asm = "\n".join([
        "\tv_mov_b32_e32 v4, v9",
        "\tv_mfma_f32_32x32x16_bf16 v[0:15], v[4:7], v[8:11], v[0:15]",
        "\tv_mov_b32_e32 v5, v9",
        "\ts_nop 1",
        "\tv_mfma_f32_32x32x16_bf16 v[0:15], v[4:7], v[8:11], v[0:15]",
        "\tv_accvgpr_write_b32 a20, v1",
        "\tv_mfma_f32_32x32x16_bf16 v[0:15], a[20:23], v[8:11], v[0:15]",
    ])
    bad = _violations(asm)
    assert len(bad) == 2 and "v_mov_b32_e32" in bad[0] and "v_accvgpr_write_b32" in bad[1]


def test_checker_flags_planted_memory_hazards():
    asm = "\n".join([
        "\tv_readlane_b32 s0, v4, 3",
        "\tv_readlane_b32 s1, v5, 3",
        "\ts_mov_b32 m0, s4",
        "\tglobal_load_lds_dwordx4 v254, s[0:1]",
        "\ts_nop 4",
        "\ts_mov_b32 m0, s5",
        "\ts_nop 0",
        "\tglobal_load_lds_dwordx4 v254, s[0:1]",
    ])
    bad = _mem_violations(asm)
    assert len(bad) == 3, bad   # M0 distance 0, s0 distance 2, s1 distance 1; the second load is clean


def test_checker_flags_a_planted_result_hazard():
    asm = "\n".join([
        "\tv_mfma_f32_16x16x32_bf16 a[0:3], v[0:3], v[4:7], a[0:3]",
        "\tv_mfma_f32_16x16x32_bf16 a[4:7], v[0:3], v[4:7], a[4:7]",
        "\tv_accvgpr_read_b32 v9, a1",
        "\ts_nop 7",
        "\tv_accvgpr_read_b32 v10, a5",
        "\tv_mfma_f32_32x32x16_bf16 v[16:31], v[0:3], v[4:7], v[16:31]",
        "\tv_mfma_f32_32x32x16_bf16 v[16:31], v[0:3], v[4:7], v[16:31]",
        "\ts_nop 10",
        "\tglobal_store_dwordx4 v40, v[16:19], off",
    ])
    bad = _result_violations(asm)
    # a1 one wait state after its MFMA; the accumulation into v[16:31] is allowed; the store
    # comes 11 wait states after the second 32x32 MFMA (12 needed); a5 is clear
    assert len(bad) == 2 and "a1" not in bad[1] and "global_store" in bad[1], bad
