"""Writes tests/golden/golden.json from data and code the reference holds.

Run in the build container (it reads the reference tree, which the GPU host
does not have):

    python tests/golden/make_golden.py [/root/reference]

Contents:
  rope     sha256 and size of the reference rope_lut.bin, and 512 entries
           decoded from it by plain bit extraction (format of
           scripts/generate_rope_lut.py:20-41, 104-150).
  kat      the expected hashes of the reference's attention known-answer test
           (_rtl_check/linear_4pe_reduction_cosim/tb_attention_pe0_kv_rtl.cpp:109-110).
  decode   outputs of the reference emulator's own attention stage
           (software_sim/llama2_decoder_sw_emulator.cpp:602-714, compiled by
           oracle/Makefile into oracle/_ref) on decode sequences whose inputs
           come from tests/helpers.py generators: per step the reference
           rotates q/k (emulator:526-541), then appends and attends.  Stored:
           the A14 codes and scales of the last step and an FNV hash chained
           over every step's A14 codes and scales.
"""
import hashlib
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(REPO, "tests"))
sys.path.insert(0, os.path.join(REPO, "oracle"))

from helpers import q17_uniform  # noqa: E402

DECODE_CASES = [
    # (seed, last position, span bits of the Q15.17 inputs)
    (7, 100, 18),
    (11, 40, 22),
    (13, 24, 30),
]


def step_inputs(seed: int, pos: int, span: int):
    base = seed * 1000003 + pos * 3
    return (q17_uniform(base + 0, (4096,), span), q17_uniform(base + 1, (4096,), span),
            q17_uniform(base + 2, (4096,), span))


def fnv_chain(h: int, data: bytes) -> int:
    for b in data:
        h ^= b
        h = (h * 1099511628211) & 0xFFFFFFFFFFFFFFFF
    return h


def decode_rope_file(buf: bytes, picks):
    bits = np.unpackbits(np.frombuffer(buf, np.uint8), bitorder="little")
    out = []
    for pos, pair in picks:
        base = ((pos * 4 + pair // 16) * 128) * 8
        lane = pair % 16

        def field(off):
            v = int((bits[base + off: base + off + 19].astype(np.int64) << np.arange(19)).sum())
            return v - (1 << 19) if v >= (1 << 18) else v

        out.append([int(pos), int(pair), field(38 * lane), field(38 * lane + 19)])
    return out


def main():
    ref_root = sys.argv[1] if len(sys.argv) > 1 else "/root/reference"
    with open(os.path.join(ref_root, "rope_lut.bin"), "rb") as f:
        lut = f.read()
    rng = np.random.default_rng(2026)
    picks = [(0, j) for j in range(64)] + [(4095, j) for j in range(64)]
    picks += [(int(p), int(j)) for p, j in zip(rng.integers(0, 4096, 384), rng.integers(0, 64, 384))]
    golden = {
        "rope": {
            "sha256": hashlib.sha256(lut).hexdigest(),
            "bytes": len(lut),
            "positions": len(lut) // 512,
            "theta": 10000.0,
            "entries": decode_rope_file(lut, picks),
        },
        "kat": {"pos0": "0xf93d262d08160f1b", "pos1": "0x79a79ee8fe403198",
                "seeds": [[3, 11, 29], [43, 61, 79]]},
        "decode": [],
    }

    import oracle as O
    cos, sin = O.rope_unpack(np.frombuffer(lut, np.uint8))
    ref = O.Reference()
    ref.set_rope(cos, sin)
    for seed, last, span in DECODE_CASES:
        cache = ref.cache(last + 1)
        h = 1469598103934665603
        for pos in range(last + 1):
            q, k, v = step_inputs(seed, pos, span)
            qr, kr = ref.apply_rope(q, pos), ref.apply_rope(k, pos)
            aq, asc = cache.attention(qr, kr, v, pos)
            h = fnv_chain(h, aq.tobytes() + asc.tobytes())
        golden["decode"].append({
            "seed": seed, "last_position": last, "span_bits": span,
            "chain_hash": hex(h),
            "a14_last": aq.astype(int).tolist(),
            "scale_last": [float(x) for x in asc],
        })
    with open(os.path.join(HERE, "golden.json"), "w") as f:
        json.dump(golden, f)
    print("wrote", os.path.join(HERE, "golden.json"))


if __name__ == "__main__":
    main()
