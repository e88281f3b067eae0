"""Writes the committed golden fixtures under tests/golden/.

ggml_dequant_q8_0.json: the q8_0 case of the reference's own golden file
fixtures/oracle/ggml_dequant.json (gguf-py 0.19.0, numpy 2.5.4; checked bit for bit by
the reference's crates/qubivex-backend-cpu/tests/oracle.rs:10-50).  The data is copied
as data (raw block bytes and the f32 bit patterns gguf-py produced); nothing is run.

Usage: python tests/golden/make_golden.py [/root/reference]
"""
import json
import os
import sys

HERE = os.path.dirname(os.path.abspath(__file__))


def main(ref="/root/reference"):
    src = os.path.join(ref, "fixtures/oracle/ggml_dequant.json")
    with open(src) as f:
        data = json.load(f)
    case = [c for c in data["cases"] if c["dtype"] == "q8_0"]
    assert len(case) == 1
    out = {
        "source": "fixtures/oracle/ggml_dequant.json (reference), case q8_0",
        "generator": data["generator"],
        "gguf": data["gguf"],
        "numpy": data["numpy"],
        "case": case[0],
    }
    with open(os.path.join(HERE, "ggml_dequant_q8_0.json"), "w") as f:
        json.dump(out, f, indent=0)


if __name__ == "__main__":
    main(*sys.argv[1:])
