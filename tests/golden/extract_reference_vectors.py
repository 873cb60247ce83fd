#!/usr/bin/env python3
"""Extract the reference's in-source known-answer vectors into a JSON fixture.

Reads (as text, never executes) the Rust unit tests of the reference and
writes tests/golden/reference_vectors.json: inputs and expected outputs only.
Run in the build container, where /root/reference exists:

    python tests/golden/extract_reference_vectors.py [/root/reference]

Sources (paths relative to the reference root):
  rust/npu-asr-host/src/lib.rs  test_bf16_round    (:876-887)
                                test_layer_norm     (:889-900)
                                test_layer_norm_normalize (:902-911)
                                test_rope           (:913-948)
                                mha_inputs + test_mha_no_round (:950-1001)
"""
import json
import os
import re
import sys

NUM = re.compile(r"[-+]?(?:\d+\.\d*|\.\d+|\d+)(?:[eE][-+]?\d+)?")


def fn_body(src, name):
    """Text of `fn name(...) ... { ... }` (brace matched)."""
    i = src.index("fn %s(" % name)
    j = src.index("{", i)
    depth = 0
    for k in range(j, len(src)):
        if src[k] == "{":
            depth += 1
        elif src[k] == "}":
            depth -= 1
            if depth == 0:
                return src[j + 1:k]
    raise ValueError(name)


def floats(text):
    # drop identifiers that contain digits (e.g. f32, arr2, 1e-4 stays)
    text = re.sub(r"\b[A-Za-z_][A-Za-z_0-9]*\b", " ", text)
    return [float(x) for x in NUM.findall(text)]


def main():
    root = sys.argv[1] if len(sys.argv) > 1 else "/root/reference"
    host = open(os.path.join(root, "rust/npu-asr-host/src/lib.rs")).read()
    out = {}

    # test_layer_norm: x[2,4], gamma[4], beta[4], eps, exp[8], tol
    v = floats(fn_body(host, "test_layer_norm"))
    assert len(v) == 8 + 4 + 4 + 1 + 8 + 1, len(v)
    out["layer_norm"] = dict(rows=2, d=4, x=v[0:8], gamma=v[8:12], beta=v[12:16],
                             eps=v[16], expected=v[17:25], tol=v[25])

    # test_layer_norm_normalize: x[2,4], eps, exp[8], tol
    v = floats(fn_body(host, "test_layer_norm_normalize"))
    assert len(v) == 8 + 1 + 8 + 1, len(v)
    out["layer_norm_normalize"] = dict(rows=2, d=4, x=v[0:8], eps=v[8],
                                       expected=v[9:17], tol=v[17])

    # test_rope: shapes (2,8) ln, (2,4) cos, (2,4) sin, call (2,4), exp[16], tol
    v = floats(fn_body(host, "test_rope"))
    # literal stream: 2,8, ln16, 2,4, cos8, 2,4, sin8, 2,4 (n_heads, head_dim), exp16, tol
    assert len(v) == 2 + 16 + 2 + 8 + 2 + 8 + 2 + 16 + 1, len(v)
    p = 0
    p += 2; ln = v[p:p + 16]; p += 16
    p += 2; cos = v[p:p + 8]; p += 8
    p += 2; sin = v[p:p + 8]; p += 8
    n_heads, head_dim = int(v[p]), int(v[p + 1]); p += 2
    exp = v[p:p + 16]; p += 16
    out["rope"] = dict(rows=2, n_heads=n_heads, head_dim=head_dim, x=ln, cos=cos,
                       sin=sin, expected=exp, tol=v[p])

    # mha_inputs: (3,8) q, (3,8) k, (3,8) v
    v = floats(fn_body(host, "mha_inputs"))
    assert len(v) == 3 * (2 + 24), len(v)
    q, k, vv = v[2:26], v[28:52], v[54:78]
    # test_mha_no_round: mha(&q,&k,&v, 2, 4, false, 3) -> exp[24], tol
    e = floats(fn_body(host, "test_mha_no_round"))
    assert len(e) == 3 + 24 + 1, len(e)
    out["mha_no_round"] = dict(t=3, n_heads=int(e[0]), head_dim=int(e[1]),
                               valid_len=int(e[2]), q=q, k=k, v=vv,
                               expected=e[3:27], tol=e[27])

    # test_bf16_round: explicit value pairs (NaN case handled by the test)
    body = fn_body(host, "test_bf16_round")
    pairs = []
    for m in re.finditer(r"assert_eq!\(bf16_round\(([^)]*)\),\s*([^)]*)\)", body):
        pairs.append((float(m.group(1)), float(m.group(2)), 0.0))
    for m in re.finditer(r"assert!\(\(bf16_round\(([^)]*)\)\s*-\s*\(?([-0-9.e]+)\)?\)\.abs\(\)\s*<\s*([0-9.e-]+)\)", body):
        pairs.append((float(m.group(1)), float(m.group(2)), float(m.group(3))))
    assert len(pairs) == 8, pairs
    out["bf16_round"] = [dict(x=a, expected=b, tol=t) for a, b, t in pairs]

    out["_source"] = "rust/npu-asr-host/src/lib.rs unit tests (text extraction)"
    dst = os.path.join(os.path.dirname(os.path.abspath(__file__)), "reference_vectors.json")
    with open(dst, "w") as f:
        json.dump(out, f, indent=1)
    print("wrote", dst)


if __name__ == "__main__":
    main()
