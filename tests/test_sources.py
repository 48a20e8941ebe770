"""Source checks that need no GPU: patterns in the HIP sources that the
ROCm 7.2 toolchain is known to miscompile."""

import re

from conftest import PKG

CSRC = PKG / "csrc"
VECTOR_TYPES = ("u32x4", "u32x2", "f32x4", "f32x16", "bf16x8", "f16x8")


# declarations, also reference parameters such as `const u32x4 (&pb)[2]`
DECL = re.compile(r"\b(?:%s)\s+\(?&?\s*(\w+)\)?((?:\s*\[[^\]]*\])*)" % "|".join(VECTOR_TYPES))
ARG = re.compile(r"__builtin_bit_cast\s*\(\s*[\w:<>]+\s*,\s*([\w.]+)((?:\[[^\]]+\])+)\s*\)")


def _decl_ranks(text, before=None):
    """Array rank of every variable or member declared with a vector type
    (``u32x4 kop[4][NDS]`` -> {"kop": 2}; a plain vector has rank 0), from
    the last declaration of each name before offset ``before`` (names are
    reused across functions)."""
    ranks = {}
    for m in DECL.finditer(text):
        if before is not None and m.start() >= before:
            break
        ranks[m.group(1)] = m.group(2).count("[")
    return ranks


def _flagged(text):
    out = []
    for m in ARG.finditer(text):
        ranks = _decl_ranks(text, m.start())
        name = m.group(1).split(".")[-1]
        subs = re.findall(r"\[([^\]]+)\]", m.group(2))
        if name not in ranks or len(subs) <= ranks[name]:
            continue  # a whole vector (an array element), or not a vector
        if subs[-1].strip() == "0":
            continue  # element 0 reads correctly
        out.append((text.count("\n", 0, m.start()) + 1, m.group(0)))
    return out


def test_no_bit_cast_of_a_vector_element():
    """``__builtin_bit_cast(T, v[i])`` with ``v`` a vector value reads element
    0 whatever i is (the generated load drops the element offset). An element
    has to go through a scalar first; index 0 reads the right element."""
    bad = []
    for path in sorted(CSRC.glob("*.hip")) + sorted(CSRC.glob("*.h")):
        bad += [f"{path.name}:{line}: {expr}" for line, expr in _flagged(path.read_text())]
    assert not bad, "bit_cast of a vector element (reads element 0):\n" + "\n".join(bad)


def test_lint_catches_the_pattern():
    """The check above flags a vector-element bit_cast and passes the safe
    forms, with names redeclared between functions."""
    text = ("u32x4 pb[2];\nu32x4 x;\n"
            "a = __builtin_bit_cast(bf16x2, pb[ks][e]);\n"   # element e of a vector: flagged
            "b = __builtin_bit_cast(bf16x8, pb[ks]);\n"      # a whole vector: fine
            "c = __builtin_bit_cast(uint32_t, x[0]);\n"      # element 0: fine
            "u32x4 pb;\n"                                    # another function's pb
            "d = __builtin_bit_cast(uint32_t, pb[3]);\n"     # element 3 of it: flagged
            "void f(const u32x4 (&pp)[2]) {\n"               # a reference parameter
            "e = __builtin_bit_cast(bf16x2, pp[1][2]);\n")   # flagged
    assert [expr for _, expr in _flagged(text)] == [
        "__builtin_bit_cast(bf16x2, pb[ks][e])", "__builtin_bit_cast(uint32_t, pb[3])",
        "__builtin_bit_cast(bf16x2, pp[1][2])"]
