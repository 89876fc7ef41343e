"""Writes tests/golden/prototxt_cases.json from the reference's test cases.

The reference's C++ op tests describe each case in a protobuf text file
(test/zoo/teco/<op>/test_case/*.prototxt): input / output tensors with shapes,
dtypes and either a seeded random_data recipe or fixed prev_value values, op
parameters (tecokernel_param) and the pass criterion (test_param).  These
files are test data; this script parses them (a small text-format reader, no
protobuf dependency) and stores the cases of the ops on this library's path
as JSON, so the replay tests can run without the reference checkout.

Run in a checkout that has the reference at /root/reference:
    python tests/golden/make_prototxt_cases.py [reference_root]
"""
import json
import os
import re
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
OPS = ["rms_norm", "reshape_and_cache", "flash_attention", "causal_conv1d", "memset"]
TOKEN = re.compile(r'\s*(?:(#[^\n]*)|("(?:[^"\\]|\\.)*")|([{}:])|([^\s{}:"]+))')


def tokens(text):
    pos = 0
    while pos < len(text):
        m = TOKEN.match(text, pos)
        if m is None or m.end() == pos:
            if text[pos:].strip() == "":
                return
            raise ValueError(f"cannot parse near: {text[pos:pos + 40]!r}")
        pos = m.end()
        if m.group(1):
            continue
        if m.group(2):
            yield ("str", m.group(2)[1:-1])
        elif m.group(3):
            yield (m.group(3), m.group(3))
        elif m.group(4):
            yield ("word", m.group(4))


def scalar(word):
    for conv in (int, float):
        try:
            return conv(word)
        except ValueError:
            pass
    if word in ("true", "false"):
        return word == "true"
    return word  # enum name


def parse_message(toks, end=None):
    """Returns {field: [values...]} (every field repeated-capable)."""
    msg = {}
    while True:
        t = next(toks, None)
        if t is None:
            if end is not None:
                raise ValueError("unterminated message")
            return msg
        if t[0] == "}":
            return msg
        if t[0] != "word":
            raise ValueError(f"field name expected, got {t}")
        name = t[1]
        t = next(toks)
        if t[0] == ":":
            t = next(toks)
        if t[0] == "{":
            val = parse_message(toks, end="}")
        elif t[0] == "str":
            val = t[1]
        else:
            val = scalar(t[1])
        msg.setdefault(name, []).append(val)


def simplify(x):
    """Single-element lists become scalars, except the repeated fields below."""
    repeated = {"input", "output", "dims", "value_i", "value_f", "value_l"}
    if isinstance(x, dict):
        return {k: [simplify(v) for v in vs] if k in repeated else simplify(vs[0])
                for k, vs in x.items()}
    return x


def load_case(path):
    with open(path) as f:
        return simplify(parse_message(tokens(f.read())))


def main():
    ref = sys.argv[1] if len(sys.argv) > 1 else "/root/reference"
    out = {}
    for op in OPS:
        d = os.path.join(ref, "test", "zoo", "teco", op, "test_case")
        cases = []
        for name in sorted(os.listdir(d)):
            if name.endswith(".prototxt"):
                c = load_case(os.path.join(d, name))
                c["file"] = f"test/zoo/teco/{op}/test_case/{name}"
                cases.append(c)
        out[op] = cases
    path = os.path.join(HERE, "prototxt_cases.json")
    with open(path, "w") as f:
        json.dump(out, f, indent=1, sort_keys=True)
    print(path, {k: len(v) for k, v in out.items()})


if __name__ == "__main__":
    main()
