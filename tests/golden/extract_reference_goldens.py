"""Extract the reference's golden vectors for this path into a JSON fixture.

Run once in the build container (it reads /root/reference as text; nothing in
the reference is imported or executed).  The output, reference_goldens.json,
is committed; tests read only the JSON, so /root/reference is not needed at
test time.

Sources (mlavergn/llama.zig):
  src/ggml/quants/golden.zig:53-133      FNV-1a of quantize_row_*_ref bytes,
                                          dequantize_row_* floats, and
                                          quantize_* chunk with/without imatrix
                                          (4 rows x 256, five patterns)
  src/ggml/cpu/quants/golden.zig:56-211  raw f32 bits of ggml_vec_dot_*_generic
                                          (512 elements, six patterns) and
                                          FNV-1a of the q8_0/q8_1/q8_K row
                                          quantizers
"""
import json
import pathlib
import re
import sys

REF = pathlib.Path(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
OUT = pathlib.Path(__file__).with_name("reference_goldens.json")

TYPES = ("Q4_0", "Q4_K", "Q5_K", "Q6_K", "Q8_0", "Q8_1", "Q8_K", "IQ4_XS")


def quant_goldens():
    src = (REF / "src/ggml/quants/golden.zig").read_text()
    rows = []
    for m in re.finditer(r"\.\{ \.name = \"(\w+)\", \.pattern = \"(\w+)\",([^\n]*)\},", src):
        name, pattern, rest = m.groups()
        if name not in TYPES:
            continue
        rec = {"name": name, "pattern": pattern}
        for key in ("type", "row_size", "ref", "deq", "chunk", "chunk_bytes", "chunk_imatrix"):
            km = re.search(r"\." + key + r" = (0x[0-9a-fA-F]+|\d+)", rest)
            if km:
                rec[key] = int(km.group(1), 0)
        rows.append(rec)
    return rows


def dot_goldens():
    src = (REF / "src/ggml/cpu/quants/golden.zig").read_text()
    out = {}
    for name in ("q8_0", "q4_0", "q4_K", "q5_K", "q6_K", "iq4_xs"):
        m = re.search(r"pub const " + name + r" = Dot\{(.*?)\};", src, re.S)
        out[name] = {k: int(v, 16) for k, v in re.findall(r"\.(\w+) = 0x([0-9A-Fa-f]+)", m.group(1))}
    rows = {}
    for name in ("row_q8_0", "row_q8_1", "row_q8_K"):
        m = re.search(r"pub const " + name + r" = Row\{(.*?)\};", src, re.S)
        rows[name] = {k: int(v, 16) for k, v in re.findall(r"\.(\w+) = 0x([0-9A-Fa-f]+)", m.group(1))}
    return out, rows


def main():
    q = quant_goldens()
    dots, rows = dot_goldens()
    doc = {
        "source": "mlavergn/llama.zig src/ggml/quants/golden.zig, src/ggml/cpu/quants/golden.zig",
        "quant": {"n_per_row": 256, "n_rows": 4, "records": q},
        "vecdot": {"nelem": 512, "dots": dots, "rows": rows},
    }
    OUT.write_text(json.dumps(doc, indent=1) + "\n")
    print(f"wrote {OUT}: {len(q)} quant records, {len(dots)} dots, {len(rows)} row quantizers")


if __name__ == "__main__":
    main()
