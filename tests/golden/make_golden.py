"""Writes the committed fixtures of tests/golden/ from the CPU oracle (oracle/gfr_oracle.c).

The reference ships no golden vectors for this path, so these fixtures are the oracle's outputs on the
reference's own known-answer procedures, frozen so that a later change to the oracle or to a kernel is caught:

  codebook.npy        all 65536 codebook states (experts.rs:43-46), uint16 fp16 bits
  tiles_k{2,3,4,5}.npz  two 16 x 32-column matrices of seeded trellis words and their decoded fp16 weights
                      (experts.rs:47-74 generalised to K bits; splitmix64 words, seed 1234 + K)
  grouping.npz        the reference probe's xorshift64 routing (grouping.rs:138-157, seed 0x0123456789abcdef,
                      E 289, 9 slots, capacity 64) for rows 1, 2, 31, 32, 33, 63, 64: picks and count / ids / members

Run: python tests/golden/make_golden.py   (needs the oracle library; writes next to this file)
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "..", "..", "oracle"))
import oracle  # noqa: E402

M64 = (1 << 64) - 1


def splitmix64_words(seed, n):
    out = np.empty(n, np.uint32)
    s = seed & M64
    for i in range(n):
        s = (s + 0x9E3779B97F4A7C15) & M64
        z = s
        z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & M64
        z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & M64
        out[i] = (z ^ (z >> 31)) & 0xFFFFFFFF
    return out


def xorshift_cases(rows_list, slots=9, seed=0x0123456789ABCDEF):
    """grouping.rs:138-157: xorshift64 per row; concentrated rows start at expert 0, spread rows at seed % 288;
    slot s picks (start + 37 s) % 288, slot 8 the shared id 288."""
    out = []
    for rows in rows_list:
        for concentrated in (True, False):
            picks = np.empty((rows, slots), np.int32)
            for r in range(rows):
                seed ^= (seed << 13) & M64
                seed ^= seed >> 7
                seed ^= (seed << 17) & M64
                start = 0 if concentrated else seed % 288
                for s in range(slots):
                    picks[r, s] = 288 if s == 8 else (start + s * 37) % 288
            out.append((rows, concentrated, picks))
    return out


def main():
    np.save(os.path.join(HERE, "codebook.npy"), oracle.codebook_table())
    for bits in (2, 3, 4, 5):
        kin, n = 32, 32
        words = splitmix64_words(1234 + bits, (kin // 16) * (n // 16) * 8 * bits)
        w = oracle.unpack(words, kin, n, bits)
        np.savez(os.path.join(HERE, f"tiles_k{bits}.npz"), words=words, kin=kin, n=n, weights=w)
    cases = xorshift_cases([1, 2, 31, 32, 33, 63, 64])
    arrs = {}
    for i, (rows, conc, picks) in enumerate(cases):
        c, ids, mem = oracle.group(picks, rows, 9, 289, 64)
        arrs[f"picks{i}"] = picks
        arrs[f"count{i}"] = np.int32(c)
        arrs[f"ids{i}"] = ids[:c]
        arrs[f"members{i}"] = mem
    np.savez_compressed(os.path.join(HERE, "grouping.npz"), n=len(cases), **arrs)
    print("wrote", sorted(os.listdir(HERE)))


if __name__ == "__main__":
    main()
