"""Writes the golden fixtures in this folder from the Reef engine's own golden vectors.

The engine ships no golden files; its golden writer (coral/host/gen_golden.cpp)
computes them at build time from the engine headers. ``make -C oracle ref``
compiles that writer from the reference checkout and runs it into
oracle/_ref/golden/*.hpp. This script reads those generated headers (data only:
seeded inputs and the engine's outputs, floats as hex literals) and stores the
cases the int8 attention path depends on as JSON, floats as IEEE-754 bit
patterns so they round-trip exactly:

  exp_nonpositive.json   math.hpp kExp            (math.hpp:34-67 on 3013 inputs)
  attention_f32.json     attention.hpp kAttention (attend_head, 7 shapes)
  int8_softmax.json      int8.hpp kInt8Softmax    (masked_softmax_int8, 3 shapes)
  int8_attention.json    int8.hpp kInt8Attention  (attend_head_int8, 7 shapes)
  exp_table.json         int8.hpp i8_exp_table    (exp_table())
  w8a8_linear.json       linear.hpp kW8a8         (quantize_rows + int32 matmul + rescale)

Run:  make -C oracle ref && python tests/golden/make_fixtures.py
"""
from __future__ import annotations

import json
import os
import re
import struct

HERE = os.path.dirname(os.path.abspath(__file__))
GEN = os.path.join(HERE, "..", "..", "oracle", "_ref", "golden")

_ARRAY = re.compile(r"inline constexpr ([\w:]+) (\w+)\[\] = \{(.*?)\};", re.S)
_TABLE = re.compile(r"inline constexpr (\w+) (\w+)\[\] = \{(.*?)\n\};", re.S)


def _bits(literal: str) -> int:
    value = float.fromhex(literal.rstrip("F"))
    return struct.unpack("<I", struct.pack("<f", value))[0]


def parse(path: str):
    text = open(path).read()
    arrays = {}
    for ctype, name, body in _ARRAY.findall(text):
        if ctype.endswith("Case"):
            continue
        items = [t.strip() for t in body.split(",") if t.strip()]
        if ctype == "float":
            arrays[name] = [_bits(t) for t in items]
        else:
            arrays[name] = [int(t.rstrip("U")) for t in items]
    tables = {}
    for ctype, name, body in _TABLE.findall(text):
        if not ctype.endswith("Case"):
            continue
        rows = re.findall(r"\{(.*?)\},", body)
        tables[name] = [[f.strip() for f in row.split(",")] for row in rows]
    return arrays, tables


def main() -> None:
    math_a, math_t = parse(os.path.join(GEN, "math.hpp"))
    n, xs, ys = math_t["kExp"][0]
    dump("exp_nonpositive.json", {"x_bits": math_a[xs], "y_bits": math_a[ys]})

    att_a, att_t = parse(os.path.join(GEN, "attention.hpp"))
    cases = []
    for row in att_t["kAttention"]:
        sq, sk, d, start, window = (int(v) for v in row[:5])
        q, k, v, y = (att_a[t] for t in row[5:9])
        cases.append(dict(query_len=sq, key_len=sk, head_dim=d, query_start=start,
                          window=window, q_bits=q, k_bits=k, v_bits=v, y_bits=y))
    dump("attention_f32.json", {"cases": cases})

    i8_a, i8_t = parse(os.path.join(GEN, "int8.hpp"))
    dump("exp_table.json", {"table": i8_a["i8_exp_table"]})
    cases = []
    for row in i8_t["kInt8Softmax"]:
        rows, n, shift = (int(v) for v in row[:3])
        cases.append(dict(rows=rows, n=n, shift=shift, scores=i8_a[row[4]],
                          probs=i8_a[row[5]]))
    dump("int8_softmax.json", {"cases": cases})
    cases = []
    for row in i8_t["kInt8Attention"]:
        sq, sk, d, start, window, sshift, oshift = (int(v) for v in row[:7])
        q, k, v, y = (i8_a[t] for t in row[8:12])
        cases.append(dict(query_len=sq, key_len=sk, head_dim=d, query_start=start,
                          window=window, score_shift=sshift, out_shift=oshift,
                          q=q, k=k, v=v, y=y))
    dump("int8_attention.json", {"cases": cases})

    lin_a, lin_t = parse(os.path.join(GEN, "linear.hpp"))
    cases = []
    for row in lin_t["kW8a8"]:
        rows, fin, fout = (int(v) for v in row[:3])
        x, wt, ws, y = (lin_a[t] for t in row[3:7])
        cases.append(dict(rows=rows, in_features=fin, out_features=fout, x_bits=x, wt=wt,
                          w_scale_bits=ws, y_bits=y))
    dump("w8a8_linear.json", {"cases": cases})


def dump(name: str, payload) -> None:
    payload = {"source": "Reef coral/host/gen_golden.cpp output, engine headers", **payload}
    with open(os.path.join(HERE, name), "w") as f:
        json.dump(payload, f, separators=(",", ":"))
    print(name, os.path.getsize(os.path.join(HERE, name)), "bytes")


if __name__ == "__main__":
    main()
