"""Build-time check of a hazard the compiler does not guard: the diagonal
Cholesky kernel (crb_amd/csrc/chol.hip) issues `v_fmac_f32_dpp` from inline
assembly, and a DPP read of a VGPR needs two wait states after the VALU
instruction that wrote it.  LLVM's hazard recognizer does not look inside
asm statements, so a VALU write of the DPP source placed right before one
of them by the register allocator or scheduler would read a stale value
(a silently wrong factor).  The asm variants that follow a fresh write
carry their own `s_nop 1`; this test compiles chol.hip for gfx950 to AMD
assembly and checks every `v_fmac_f32_dpp` of the build: within the two
wait states before it (each instruction 1, `s_nop N` N + 1) no VALU
instruction writes its DPP source and no label (another path in) appears.
CPU only: it needs hipcc, not a GPU."""
import os
import re
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")


def _regs(tok):
    """VGPR numbers named by an operand token (v7, v[4:7]); empty for others."""
    tok = tok.strip().lstrip("-")
    m = re.fullmatch(r"v(\d+)", tok)
    if m:
        return {int(m.group(1))}
    m = re.fullmatch(r"v\[(\d+):(\d+)\]", tok)
    if m:
        return set(range(int(m.group(1)), int(m.group(2)) + 1))
    return set()


def _operands(line):
    parts = line.split(None, 1)
    if len(parts) < 2:
        return parts[0], []
    ops = re.split(r",\s*", parts[1].split(" row_")[0].split(" quad_perm")[0])
    return parts[0], [o.strip() for o in ops]


def hazards(asm_text):
    """Lines of `v_fmac_f32_dpp` instructions whose DPP source may have been
    written by a VALU instruction less than two wait states before."""
    seq = []                       # ("label", name) or ("inst", text)
    for raw in asm_text.splitlines():
        s = raw.split(";")[0].strip()
        if not s or s.startswith("."):
            continue
        if s.endswith(":"):
            seq.append(("label", s))
        else:
            seq.append(("inst", s))
    bad = []
    for i, (kind, text) in enumerate(seq):
        if kind != "inst" or not text.startswith("v_fmac_f32_dpp"):
            continue
        _, ops = _operands(text)
        src = _regs(ops[1])
        ws, j = 0, i - 1
        while ws < 2 and j >= 0:
            k2, t2 = seq[j]
            if k2 == "label":
                bad.append((text, f"label {t2} within the hazard window"))
                break
            mn, o2 = _operands(t2)
            if mn == "s_nop":
                ws += int(o2[0], 0) + 1
            else:
                if mn.startswith("v_") and o2 and _regs(o2[0]) & src:
                    bad.append((text, f"written by '{t2}' {ws} wait states before"))
                    break
                ws += 1
            j -= 1
    return bad


def test_hazard_checker_finds_a_planted_hazard():
    """The checker itself: a DPP read right after a write of its source is
    found; one behind `s_nop 1` or behind two other instructions is not."""
    planted = "\n".join([
        "\tv_mul_f32_e32 v38, v1, v2",
        "\tv_fmac_f32_dpp v13, -v38, v38 row_newbcast:1 row_mask:0xf bank_mask:0xf bound_ctrl:1",
    ])
    assert len(hazards(planted)) == 1
    ok1 = "\n".join([
        "\tv_mul_f32_e32 v38, v1, v2",
        "\ts_nop 1",
        "\tv_fmac_f32_dpp v13, -v38, v38 row_newbcast:1 row_mask:0xf bank_mask:0xf bound_ctrl:1",
    ])
    ok2 = "\n".join([
        "\tv_mul_f32_e32 v38, v1, v2",
        "\tv_add_f32_e32 v40, v1, v2",
        "\tv_add_f32_e32 v41, v1, v2",
        "\tv_fmac_f32_dpp v13, -v38, v38 row_newbcast:1 row_mask:0xf bank_mask:0xf bound_ctrl:1",
    ])
    assert hazards(ok1) == [] and hazards(ok2) == []
    wide = "\n".join([
        "\tv_pk_mov_b32 v[36:37], v[2:3], v[2:3] op_sel:[0,1]",
        "\tv_fmac_f32_dpp v13, -v37, v38 row_newbcast:1 row_mask:0xf bank_mask:0xf bound_ctrl:1",
    ])
    assert len(hazards(wide)) == 1


@pytest.mark.skipif(not shutil.which(HIPCC) and not os.path.exists(HIPCC),
                    reason="hipcc not installed")
def test_chol_dpp_fmac_wait_states(tmp_path):
    from crb_amd.build import FLAGS
    out = tmp_path / "chol.s"
    cmd = [HIPCC, *[f for f in FLAGS if f != "-fPIC"], "--cuda-device-only", "-S",
           os.path.join(ROOT, "crb_amd", "csrc", "chol.hip"), "-o", str(out)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-2000:]
    text = out.read_text()
    n = sum(1 for ln in text.splitlines() if "v_fmac_f32_dpp" in ln)
    assert n > 0
    bad = hazards(text)
    assert not bad, bad[:5]
