"""Writes dequant_kats.json and f16_kats.json: the one-block dequantisation
known-answer vectors of internal/gguf/gguf_test.go:190-309 and the f16 decode
table of :155-186 (inputs and expected outputs as data)."""
import json
import os

HERE = os.path.dirname(os.path.abspath(__file__))


def blk(n, setters):
    b = [0] * n
    for i, v in setters:
        b[i] = v
    return b


def main():
    kats = [
        {"name": "Q4_0", "type": 2,
         "block": blk(18, [(1, 0x3C), (2, 0x9A)] + [(i, 0x88) for i in range(3, 18)]),
         "expect": {"0": 2.0, "1": 1.0, **{str(i): 0.0 for i in range(2, 32)}}},
        {"name": "Q4_1", "type": 3, "block": blk(20, [(1, 0x3C), (3, 0x38), (4, 0x23)]),
         "expect": {"0": 3.5, "1": 2.5, **{str(i): 0.5 for i in range(2, 32)}}},
        {"name": "Q5_0", "type": 6,
         "block": blk(22, [(1, 0x3C), (2, 0x03), (6, 0x04)] + [(i, 0x88) for i in range(7, 22)]),
         "expect": {"0": 4.0, "1": 0.0, "2": -8.0}},
        {"name": "Q5_1", "type": 7, "block": blk(24, [(1, 0x3C), (8, 0x4F)]), "expect": {"0": 15.0, "1": 4.0}},
        {"name": "Q8_0", "type": 8, "block": blk(34, [(1, 0x40), (2, 1), (3, 0xFF), (4, 2), (5, 0xFE)]),
         "expect": {"0": 2.0, "1": -2.0, "2": 4.0, "3": -4.0, **{str(i): 0.0 for i in range(4, 32)}}},
    ]
    with open(os.path.join(HERE, "dequant_kats.json"), "w") as f:
        json.dump(kats, f, indent=1)
    f16 = [("zero", 0x0000, "0x00000000"), ("neg-zero", 0x8000, "0x80000000"), ("one", 0x3C00, "0x3f800000"),
           ("two", 0x4000, "0x40000000"), ("neg-one", 0xBC00, "0xbf800000"), ("half", 0x3800, "0x3f000000"),
           ("inf", 0x7C00, "0x7f800000"), ("neg-inf", 0xFC00, "0xff800000"),
           ("subnormal-min", 0x0001, "0x33800000"), ("subnormal-max", 0x03FF, "0x387fc000")]
    with open(os.path.join(HERE, "f16_kats.json"), "w") as f:
        json.dump([{"name": n, "h": h, "f32_bits": b} for n, h, b in f16], f, indent=1)


if __name__ == "__main__":
    main()
