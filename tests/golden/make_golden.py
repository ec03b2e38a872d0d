"""Writes the golden fixtures (data only):

- golden_blocks.json: the golden blocks of kapel-ref/src/golden.rs
  (SplitMix64 bytes with f16 scales written at their offsets) and their
  values by the GGML-order transcriptions in tests/test_oracle.py: block
  bytes and expected values;
- iq_tables.json: the two tables of the non-linear formats, the numbers of
  kapel-core/src/iq.rs:7-78 read as text (written only where the reference's
  sources are present).

    python tests/golden/make_golden.py
"""
import json
import os
import re
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))
sys.path.insert(0, os.path.join(os.path.dirname(os.path.dirname(HERE)), "oracle"))

import test_oracle as t  # noqa: E402

Q4_1, Q5_0, Q5_1, Q4K, Q5K, Q6K, Q2K, Q3K = 4, 5, 6, 7, 8, 9, 13, 14
IQ4_NL, IQ4_XS, IQ3_S = 10, 11, 12
IQ_RS = "/root/reference/crates/kapel-core/src/iq.rs"


def iq_tables():
    """The numbers between the brackets of IQ4NL_VALUES and IQ3S_GRID."""
    if not os.path.exists(IQ_RS):
        return None
    with open(IQ_RS) as f:
        text = f.read()

    def table(name):
        body = re.search(name + r": \[[^\]]*\] = \[([^\]]*)\]", text).group(1)
        return [int(v, 0) for v in re.findall(r"-?(?:0x[0-9a-fA-F]+|\d+)", body)]

    values, grid = table("IQ4NL_VALUES"), table("IQ3S_GRID")
    assert len(values) == 16 and len(grid) == 512
    return {"source": "kapel-core/src/iq.rs", "iq4nl_values": values, "iq3s_grid": grid}


def main():
    cases = []

    def add(name, fmt, data, values):
        cases.append({"name": name, "format": fmt, "bytes": bytes(data).hex(),
                      "values": [float(v) for v in values]})

    d = t.golden_block(20, 1, [(0, t.HALF), (2, t.MINUS_ONE_AND_HALF)])
    qs = d[4:]
    add("q4_1", Q4_1, d, [float(qs[j] & 15) * 0.5 - 1.5 for j in range(16)] +
        [float(qs[j] >> 4) * 0.5 - 1.5 for j in range(16)])
    d = t.golden_block(22, 2, [(0, t.HALF)])
    add("q5_0", Q5_0, d, t.ggml_q5(d, 0.5, None))
    d = t.golden_block(24, 3, [(0, t.QUARTER), (2, t.MINUS_ONE_AND_HALF)])
    add("q5_1", Q5_1, d, t.ggml_q5(d, 0.25, -1.5))
    d = t.golden_block(84, 4, [(80, t.HALF), (82, t.QUARTER)])
    add("q2_k", Q2K, d, t.ggml_q2k(d, 0.5, 0.25))
    d = t.golden_block(110, 5, [(108, t.TWO)])
    add("q3_k", Q3K, d, t.ggml_q3k(d, 2.0))
    d = t.golden_block(144, 6, [(0, t.QUARTER), (2, t.HALF)])
    add("q4_k", Q4K, d, t.ggml_q4k(d, 0.25, 0.5))
    d = t.golden_block(176, 7, [(0, t.HALF), (2, t.QUARTER)])
    add("q5_k", Q5K, d, t.ggml_q5k(d, 0.5, 0.25))
    d = t.golden_block(210, 8, [(208, t.HALF)])
    add("q6_k", Q6K, d, t.ggml_q6k(d, 0.5))
    d = t.golden_block(18, 9, [(0, t.HALF)])
    add("iq4_nl", IQ4_NL, d, t.ggml_iq4_nl(d, 0.5))
    d = t.golden_block(136, 10, [(0, t.QUARTER)])
    add("iq4_xs", IQ4_XS, d, t.ggml_iq4_xs(d, 0.25))
    d = t.golden_block(110, 11, [(0, t.HALF)])
    add("iq3_s", IQ3_S, d, t.ggml_iq3_s(d, 0.5))
    with open(os.path.join(HERE, "golden_blocks.json"), "w") as f:
        json.dump(cases, f, indent=0)
    print(len(cases), "golden blocks")
    tables = iq_tables()
    if tables is not None:
        with open(os.path.join(HERE, "iq_tables.json"), "w") as f:
            json.dump(tables, f)
        print("iq tables")


if __name__ == "__main__":
    main()
