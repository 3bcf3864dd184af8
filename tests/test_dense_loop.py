"""The generated main loop of dense_pipe_kernel (csrc/gen_dense_loop.py -> csrc/dense_loop.inc),
checked on the CPU against the contract the kernel's inline-asm statement relies on.

The loop is one inline-asm statement over physical registers: the compiler knows only the
operands bound by register constraints (outputs, inputs) and the clobber list
(WDRZ_PIPE_CLOBBERS in csrc/attn_dense.hip). A register the loop writes that is neither an
output nor clobbered would silently corrupt a value the compiler keeps there; an input operand
written by the loop would break the values the kernel reuses after it. These tests parse every
generated instruction and check that contract, the committed macro file against the generator,
and the generator's own hazard check.
"""
import importlib.util
import re
from pathlib import Path

import pytest

CSRC = Path(__file__).resolve().parent.parent / "whisperdrz_amd" / "csrc"


def _gen():
    spec = importlib.util.spec_from_file_location("gen_dense_loop", CSRC / "gen_dense_loop.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def _macros(text):
    """{macro name: [instruction or label, ...]} from the generated file."""
    out, cur = {}, None
    for line in text.splitlines():
        m = re.match(r"#define (WDRZ_DENSE_LOOP_\w+) \\$", line)
        if m:
            cur = m.group(1)
            out[cur] = []
            continue
        m = re.match(r'\s+"(.*)\\n" \\$', line)
        if cur and m:
            out[cur].append(m.group(1).strip())
    return out


def _regs(tok):
    """Registers named by one operand token (v5, v[0:15], a[96:99], s74, m0, vcc)."""
    tok = tok.rstrip(",")
    m = re.fullmatch(r"([vas])\[(\d+):(\d+)\]", tok)
    if m:
        return {f"{m.group(1)}{i}" for i in range(int(m.group(2)), int(m.group(3)) + 1)}
    if re.fullmatch(r"[vas]\d+", tok) or tok in ("m0", "vcc"):
        return {tok}
    return set()


_NO_DEST = ("s_cmp", "s_branch", "s_cbranch", "s_nop", "s_waitcnt", "s_barrier", "buffer_load_dwordx4")


def _written(ins):
    """Registers an instruction writes (the mnemonics the generator emits)."""
    parts = ins.replace(",", " ").split()
    op, args = parts[0], parts[1:]
    if op.startswith(_NO_DEST):
        # buffer_load ... lds: the first operand is the lane's byte offset, the data goes to LDS
        return set()
    if op.startswith("v_cmp"):
        return {"vcc"}
    if op == "v_permlane32_swap_b32":
        return _regs(args[0]) | _regs(args[1])
    return _regs(args[0])


def _clobbers():
    src = (CSRC / "attn_dense.hip").read_text()
    m = re.search(r"#define WDRZ_PIPE_CLOBBERS \\\n(.*?)\n\n", src, re.S)
    assert m, "WDRZ_PIPE_CLOBBERS not found"
    return set(re.findall(r'"([^"]+)"', m.group(1)))


def _operands():
    """(outputs, inputs) register sets bound by the asm statement's constraints."""
    src = (CSRC / "attn_dense.hip").read_text()
    m = re.search(r"#define WDRZ_PIPE_OPERANDS\b(.*?): WDRZ_PIPE_CLOBBERS", src, re.S)
    assert m, "WDRZ_PIPE_OPERANDS not found"
    body = m.group(1)
    outs, ins = set(), set()
    for kind, reg in re.findall(r'"([=+]?)\{([^}]+)\}"', body):
        (outs if kind in ("=", "+") else ins).update(_regs(reg))
    return outs, ins


def test_committed_macros_match_the_generator():
    assert (CSRC / "dense_loop.inc").read_text() == _gen().render()


def test_loop_writes_only_outputs_and_clobbered_registers():
    allowed_out, inputs = _operands()
    clob = _clobbers()
    allowed = allowed_out | clob
    # the read-write operand (row offsets) is both; everything else bound as input is read-only
    read_only = inputs - allowed_out
    assert "a96" in read_only and "v136" in read_only and "v224" in read_only
    for name, body in _macros((CSRC / "dense_loop.inc").read_text()).items():
        for ins in body:
            if not ins or ins.endswith(":"):
                continue
            op = ins.split()[0]
            if not op.startswith(_NO_DEST) and not op.startswith("v_cmp"):
                assert not ins.split()[1].startswith("%"), f"{name}: writes an operand placeholder: {ins!r}"
            w = _written(ins)
            assert not (w & read_only), f"{name}: writes an input operand: {ins!r}"
            assert w <= allowed, f"{name}: writes {sorted(w - allowed)} outside outputs/clobbers: {ins!r}"


def test_labels_are_unique_per_statement():
    for name, body in _macros((CSRC / "dense_loop.inc").read_text()).items():
        labels = [x[:-1] for x in body if x.endswith(":")]
        assert labels and len(labels) == len(set(labels)), name
        assert all(lb.endswith("_%=") for lb in labels), name  # %= makes them unique per asm instance
        targets = {x.split()[1] for x in body if x.split()[0].startswith(("s_branch", "s_cbranch"))}
        assert targets <= set(labels), f"{name}: branch to an undefined label {sorted(targets - set(labels))}"


def test_generator_hazard_check_catches_a_forwarded_exp():
    gen = _gen()
    gen.check_trans_hazards(["v_exp_f32 v120, v0", "s_nop 0", "v_add_f32 v184, v120, v121"])
    with pytest.raises(AssertionError):
        gen.check_trans_hazards(["v_exp_f32 v120, v0", "v_add_f32 v184, v120, v121"])
