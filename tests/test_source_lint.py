"""Source checks on the HIP kernels that the compiler cannot make for us.

The compiler's hazard pass does not treat an inline-asm instruction as a
vector-memory store. On gfx950 a VALU write to the data registers of a store
wider than 8 bytes needs two wait states after the store; a store written
as inline asm must therefore carry its own `s_nop 1`, or the compiler may
overwrite the data registers in the next instruction and the store writes
the new values.
"""
import os
import re

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "..", "iree-hexagon-plugins_amd", "csrc")

WIDE_STORE = re.compile(r"(global|buffer|flat)_store_dwordx[34]")


def _asm_strings(text):
    """Yield (line number, concatenated string literals) of every asm
    statement in `text`."""
    for m in re.finditer(r"\basm\s+(volatile\s*)?\(", text):
        start = m.end()
        depth, i = 1, start
        while depth and i < len(text):
            depth += {"(": 1, ")": -1}.get(text[i], 0)
            i += 1
        body = text[start:i]
        # the template is the leading run of string literals
        lits = []
        for s in re.finditer(r'"((?:[^"\\]|\\.)*)"', body):
            prefix = body[:s.start()].strip()
            if prefix and not prefix.endswith('"') and lits:
                break
            lits.append(s.group(1))
        yield text.count("\n", 0, m.start()) + 1, "".join(lits)


# `s_nop N` waits N + 1 states: two need N >= 1.
NOP = re.compile(r"s_nop\s+(0x[0-9a-fA-F]+|\d+)")


def _uncovered_stores(tmpl):
    """The wide stores of one asm template whose next instruction is not an
    s_nop of at least two wait states."""
    bad = []
    for m in WIDE_STORE.finditer(tmpl):
        rest = re.split(r"\\n|\n|;", tmpl[m.end():], maxsplit=1)
        following = rest[1].strip().lstrip("\\t").strip() if len(rest) > 1 \
            else ""
        nop = NOP.match(following)
        if not nop or int(nop.group(1), 0) < 1:
            bad.append(m.group(0))
    return bad


def test_inline_asm_wide_stores_carry_wait_states():
    offenders = []
    for name in sorted(os.listdir(CSRC)):
        if not name.endswith((".hip", ".h", ".cpp")):
            continue
        with open(os.path.join(CSRC, name)) as f:
            text = f.read()
        for line, tmpl in _asm_strings(text):
            if _uncovered_stores(tmpl):
                offenders.append(f"{name}:{line}: {tmpl!r}")
    assert not offenders, ("wide inline-asm stores not followed by s_nop 1 "
                           "or more:\n" + "\n".join(offenders))


def test_lint_flags_a_bare_wide_store():
    # The checker itself: a bare dwordx4 store, and one followed by s_nop 0
    # (a single wait state), are found; s_nop 1 and more are not.
    def tmpl(tail):
        (_, t), = _asm_strings('asm volatile("global_store_dwordx4 %0, %1, '
                               'off sc1' + tail + '" ::"v"(p), "v"(v));')
        return t
    assert _uncovered_stores(tmpl(""))
    assert _uncovered_stores(tmpl("\\n\\ts_nop 0"))
    assert _uncovered_stores(tmpl("\\n\\tv_mov_b32 v0, 0\\n\\ts_nop 1"))
    assert not _uncovered_stores(tmpl("\\n\\ts_nop 1"))
    assert not _uncovered_stores(tmpl("\\n s_nop 2"))
    assert not _uncovered_stores(tmpl("\\n\\ts_nop 0x3"))
