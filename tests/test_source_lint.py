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


def test_inline_asm_wide_stores_carry_wait_states():
    offenders = []
    for name in sorted(os.listdir(CSRC)):
        if not name.endswith((".hip", ".h", ".cpp")):
            continue
        with open(os.path.join(CSRC, name)) as f:
            text = f.read()
        for line, tmpl in _asm_strings(text):
            for m in WIDE_STORE.finditer(tmpl):
                if "s_nop" not in tmpl[m.end():]:
                    offenders.append(f"{name}:{line}: {tmpl!r}")
    assert not offenders, "wide inline-asm stores without s_nop:\n" + \
        "\n".join(offenders)


def test_lint_flags_a_bare_wide_store():
    # The checker itself: a bare dwordx4 store is found, one with the
    # trailing s_nop is not.
    bad = 'asm volatile("global_store_dwordx4 %0, %1, off sc1" ::"v"(p), "v"(v));'
    good = ('asm volatile("global_store_dwordx4 %0, %1, off sc1\\n\\ts_nop 1"'
            ' ::"v"(p), "v"(v));')
    (_, t_bad), = _asm_strings(bad)
    (_, t_good), = _asm_strings(good)
    assert WIDE_STORE.search(t_bad) and "s_nop" not in t_bad
    assert WIDE_STORE.search(t_good) and "s_nop" in t_good
