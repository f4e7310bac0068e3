"""Writes tests/golden/quant_kat.json: hand-derived known-answer vectors for the
ggml block quantizers, activation quantizers, fp16 conversion and block dots.

Every expected value below is written out literally and derived by hand in
the comment beside it from the published ggml definitions (ggml-quants.c
quantize_row_*_ref, the x86 AVX2 quantize_row_q8_0/q8_1, ggml-common.h block
layouts).  Inputs are chosen so that the scales are exact powers of two and
every product is exact, which makes the rounding decisions visible:
  * ties x.5 separate round-half-even (x86 activation path) from
    roundf half-away (the _ref quantizer and all weight quantizers);
  * Q4_0 picks the signed value of largest |x| (first occurrence) and
    d = max / -8, so a positive max gives a negative d;
  * Q4_0 of an all-zero block stores d = -0.0 (0x8000) and nibbles 8;
  * Q4_1 of a constant block stores d = 0, m = x, nibbles 0.
No code from the oracle or the reference is executed to make this file.

Run:  python tests/golden/make_quant_kat.py
"""
import json
import os

Z = [0.0]


def pad(v, n=32):
    return list(v) + [0.0] * (n - len(v))


kat = {"description": __doc__.strip().splitlines()[0], "fp16": [], "q8_act": [], "q4_0": [], "q4_1": [],
       "dot": []}

# ---------------------------------------------------------------- fp16 (IEEE binary16, RNE)
kat["fp16"] = [
    # [float32 input as hex bits, expected fp16 bits]
    ["0x3f800000", "0x3c00"],  # 1.0
    ["0xbf800000", "0xbc00"],  # -1.0
    ["0x80000000", "0x8000"],  # -0.0
    ["0x477fe000", "0x7bff"],  # 65504, max finite
    ["0x477fefff", "0x7bff"],  # just below 65520 -> rounds down
    ["0x477ff000", "0x7c00"],  # 65520 = midpoint 65504/65536, tie to even -> inf
    ["0x33800000", "0x0001"],  # 2^-24, smallest subnormal
    ["0x33000000", "0x0000"],  # 2^-25 = half the smallest subnormal, tie to even -> 0
    ["0x33c00000", "0x0002"],  # 3*2^-25 = 1.5 subnormal steps, tie to even -> 2
    ["0x38800000", "0x0400"],  # 2^-14, smallest normal
    ["0x387fc000", "0x03ff"],  # 2^-14 - 2^-24, largest subnormal
    ["0x3f801000", "0x3c00"],  # 1 + 2^-11: tie between 0x3c00 and 0x3c01 -> even 0x3c00
    ["0x3f803000", "0x3c02"],  # 1 + 3*2^-11: tie between 0x3c01 and 0x3c02 -> even 0x3c02
    ["0x3f801001", "0x3c01"],  # just above the first tie -> up
    ["0x3dcccccd", "0x2e66"],  # 0.1f -> 0x2e66 (0.0999755859375)
    ["0x7f800000", "0x7c00"],  # +inf
    ["0x47800000", "0x7c00"],  # 65536 -> inf
]

# ---------------------------------------------------------------- Q8_0 / Q8_1 activations
# Block "ties_d1": amax = 127 -> d = 127/127 = 1.0 (0x3c00); id = 1 in both variants,
# so q = round(x) and only the tie rule differs.
ties_x = [127.0, 0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 126.5, 3.0, -3.0, 0.25, -0.75, 64.5, -64.5, 100.49, 0.0]
kat["q8_act"].append({
    "name": "ties_d1",
    "x": pad(ties_x),
    "d": "0x3c00",
    # rint (half to even):
    "qs_x86": pad([127, 0, 2, 2, 0, -2, -2, 126, 3, -3, 0, -1, 64, -64, 100, 0]),
    # roundf (half away from zero):
    "qs_ref": pad([127, 1, 2, 3, -1, -2, -3, 127, 3, -3, 0, -1, 65, -65, 100, 0]),
    # Q8_1 s = fp16(d * sum q): x86 sum 352 -> 0x5d80 (352 = 1.375*2^8); ref sum 353 -> 0x5d84
    "s_x86": "0x5d80",
    "s_ref": "0x5d84",
})
# Block "half_scale": amax = 63.5 -> d = 0.5 (0x3800), id = 127/63.5 = 1/0.5 = 2.
# x*id = [-127, 62.5, -62.5, 0.5, 20, 0...]
kat["q8_act"].append({
    "name": "half_scale",
    "x": pad([-63.5, 31.25, -31.25, 0.25, 10.0]),
    "d": "0x3800",
    "qs_x86": pad([-127, 62, -62, 0, 20]),
    "qs_ref": pad([-127, 63, -63, 1, 20]),
    # sums: x86 -107 -> s = -53.5 = -(1.671875*2^5) -> 0xd2b0; ref -106 -> -53.0 -> 0xd2a0
    "s_x86": "0xd2b0",
    "s_ref": "0xd2a0",
})
# All-zero block: amax 0 -> d = 0, id = 0, q = 0, s = 0.
kat["q8_act"].append({
    "name": "zero",
    "x": pad([]),
    "d": "0x0000",
    "qs_x86": pad([]),
    "qs_ref": pad([]),
    "s_x86": "0x0000",
    "s_ref": "0x0000",
})

# ---------------------------------------------------------------- Q4_0 (weights, _ref)
# Block "neg_max": the largest |x| is x0 = -8 -> max = -8, d = -8/-8 = 1.0 (0x3c00), id = 1.
# q = min(15, (int8)(x + 8.5)):  -8->0, 1->9, 7->15, 7.5->16->15, -7.6->0.9->0, 0.4->8,
# -0.6->7, 3.5->12, 0->8;  x16 = -2 -> 6, x31 = 6 -> 14.
# qs[j] = q[j] | q[j+16] << 4.
neg_max_x = pad([-8.0, 1.0, 7.0, 7.5, -7.6, 0.4, -0.6, 3.5])
neg_max_x[16] = -2.0
neg_max_x[31] = 6.0
kat["q4_0"].append({
    "name": "neg_max",
    "x": neg_max_x,
    "d": "0x3c00",
    "qs": [0x60, 0x89, 0x8F, 0x8F, 0x80, 0x88, 0x87, 0x8C, 0x88, 0x88, 0x88, 0x88, 0x88, 0x88, 0x88, 0xE8],
    # dequant (q-8)*d: element 3 (x=7.5) clips to 7, element 31 (x=6) -> 6
    "deq": [-8.0, 1.0, 7.0, 7.0, -8.0, 0.0, -1.0, 4.0] + [0.0] * 8 + [-2.0] + [0.0] * 14 + [6.0],
})
# Block "pos_max": |4| == |-4|, the first (x0 = +4) wins -> max = 4, d = 4/-8 = -0.5 (0xb800),
# id = -2.  q = (int8)(x*-2 + 8.5): 4->0, -4->16.5->15, 0->8, 1->6, -1.25->11, 2.2->4.
kat["q4_0"].append({
    "name": "pos_max",
    "x": pad([4.0, -4.0, 0.0, 1.0, -1.25, 2.2]),
    "d": "0xb800",
    "qs": [0x80, 0x8F, 0x88, 0x86, 0x8B, 0x84] + [0x88] * 10,
    "deq": [4.0, -3.5, 0.0, 1.0, -1.5, 2.0] + [0.0] * 26,
})
# All-zero block: max stays 0.0f, d = 0.0f/-8 = -0.0 (0x8000), id = 0, q = 8.
kat["q4_0"].append({
    "name": "zero",
    "x": pad([]),
    "d": "0x8000",
    "qs": [0x88] * 16,
    "deq": [0.0] * 32,
})

# ---------------------------------------------------------------- Q4_1 (weights, _ref)
# Block "unit": min 0, max 15 -> d = 1 (0x3c00), m = 0 (0x0000), id = 1.
# q = min(15, (int8)(x + 0.5)): 0->0, 15->15, 7.5->8, 14.6->15, 0.49->0, 3->3, 12.5->13, 1->1.
unit_x = [0.0, 15.0, 7.5, 14.6, 0.49, 3.0] + [1.0] * 10 + [12.5] + [1.0] * 15
kat["q4_1"].append({
    "name": "unit",
    "x": unit_x,
    "d": "0x3c00",
    "m": "0x0000",
    "qs": [0xD0, 0x1F, 0x18, 0x1F, 0x10, 0x13] + [0x11] * 10,
})
# Constant block: min = max = 3.25 -> d = 0, m = fp16(3.25) = 0x4280, q = (int8)(0.5) = 0.
kat["q4_1"].append({
    "name": "constant",
    "x": [3.25] * 32,
    "d": "0x0000",
    "m": "0x4280",
    "qs": [0x00] * 16,
})
# Block "neg_min": min -2, max 5.5 -> d = 7.5/15 = 0.5 (0x3800), m = -2 (0xc000), id = 2.
# q = (int8)((x+2)*2 + 0.5): -2->0, 5.5->15, 0->4, 1.3->7.
kat["q4_1"].append({
    "name": "neg_min",
    "x": pad([-2.0, 5.5, 0.0, 1.3]),
    "d": "0x3800",
    "m": "0xc000",
    "qs": [0x40, 0x4F, 0x44, 0x47] + [0x44] * 12,
})

# ---------------------------------------------------------------- block dots (raw block bytes)
# Q8_0 . Q8_0: w d=1.0, qs 1..32; a d=0.5, qs all 1 -> isum = 528, dot = 264.
kat["dot"].append({"type": "q8_0", "w_d": "0x3c00", "w_qs": list(range(1, 33)),
                   "a_d": "0x3800", "a_qs": [1] * 32, "isum": 528, "dot": 264.0})
# Q4_0 . Q8_0: w d=1.0, bytes 0x9a: low nibble 10 -> 2 (elements 0..15), high 9 -> 1 (16..31);
# a d=2.0, qs = 0..31 -> isum = 2*120 + 376 = 616, dot = 1232.
kat["dot"].append({"type": "q4_0", "w_d": "0x3c00", "w_qs": [0x9A] * 16,
                   "a_d": "0x4000", "a_qs": list(range(32)), "isum": 616, "dot": 1232.0})
# Q4_1 . Q8_1: w d=0.5, m=1.0, bytes 0x21: low 1 (0..15), high 2 (16..31);
# a d=1.0, s=4.0, qs all 1 -> isum = 48, dot = 0.5*1*48 + 1.0*4.0 = 28.
kat["dot"].append({"type": "q4_1", "w_d": "0x3800", "w_m": "0x3c00", "w_qs": [0x21] * 16,
                   "a_d": "0x3c00", "a_s": "0x4400", "a_qs": [1] * 32, "isum": 48, "dot": 28.0})

if __name__ == "__main__":
    out = os.path.join(os.path.dirname(os.path.abspath(__file__)), "quant_kat.json")
    with open(out, "w") as f:
        json.dump(kat, f, indent=1)
    print("wrote", out)
