#!/usr/bin/env python3
"""Write tests/golden/ref_hash.json: known answers of the reference's counter
hash (src/hash.c:5-13, mda_hash_mix and mda_hash_u64), computed by the
reference's own hash.c compiled from its source by oracle/Makefile
(`make -C oracle ref` -> oracle/_ref/libref_hash.so).

The synthetic-input generator of this build is defined on top of that hash,
so these vectors pin both the CPU oracle's and the GPU fill kernel's hash to
the reference bit for bit.  Run in the container that has /root/reference:
    make -C oracle ref && python tests/golden/make_golden.py
"""
import json
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, REPO)


def main():
    subprocess.run(["make", "-s", "-C", os.path.join(REPO, "oracle"), "ref"], check=True)
    from oracle import oracle as orc
    ref = orc.ref_hash_lib()
    if ref is None:
        raise SystemExit("oracle/_ref/libref_hash.so is missing (needs /root/reference)")
    mask = (1 << 64) - 1
    mix_in = [0, 1, 2, 0x9E3779B97F4A7C15, mask, 0x0123456789ABCDEF, 1 << 63, 12345678901234567]
    triples = []
    for stream in [0, 1, 2, 3, 4, 5, 6, 7, 4242]:
        for key in [0, 1, 7, 0xFFFFFFFF, mask]:
            for i in [0, 1, 2, 3, 1000, 123456789, (1 << 40) + 17, mask]:
                triples.append([stream, key, i])
    out = {
        "source": "reference src/hash.c (mda_hash_mix, mda_hash_u64) compiled by oracle/Makefile",
        "mix": [[x, ref.mda_hash_mix(x)] for x in mix_in],
        "u64": [[s, k, i, ref.mda_hash_u64(s, k, i)] for s, k, i in triples],
    }
    path = os.path.join(HERE, "ref_hash.json")
    with open(path, "w") as f:
        json.dump(out, f, separators=(",", ":"))
        f.write("\n")
    print("wrote %s (%d mix, %d u64 vectors)" % (path, len(out["mix"]), len(out["u64"])))


if __name__ == "__main__":
    main()
