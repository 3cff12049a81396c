"""The composite (boolean-output) SUF gates of the tests: the same two gates
oracle/ref_suf_eval.cpp builds with the reference's types, in the spec form
of suf_amd.composite and oracle/suf_ref.py.

MIXED: four pieces split at 2^62, 2^63, 2^63 + 2^62, one arithmetic word
and two boolean outputs over the four predicate kinds, with AND, OR, NOT,
XOR and constants.  DRELU: the ReLU gate's sign output
(include/gates/relu_gate.hpp:9-44): true on [0, 2^63), false above."""
T62, T63 = 1 << 62, 1 << 63

MIXED = {
    "alpha": [0, T62, T63, T63 + T62],
    "preds": [("lt", 1000), ("ltlow", 12, 2048), ("msb",), ("msb_add", 5000)],
    "pieces": [
        {"arith": [7], "bools": [("and", ("var", 0), ("not", ("var", 1))),
                                 ("or", ("var", 2), ("var", 3))]},
        {"arith": [11], "bools": [("xor", ("var", 1), ("var", 3)), ("const", 1)]},
        {"arith": [13], "bools": [("not", ("var", 0)),
                                  ("and", ("or", ("var", 1), ("var", 2)), ("var", 3))]},
        {"arith": [17], "bools": [("const", 0), ("var", 2)]},
    ],
}

DRELU = {
    "alpha": [0, T63],
    "preds": [],
    "pieces": [{"arith": [1], "bools": [("const", 1)]},
               {"arith": [0], "bools": [("const", 0)]}],
}
