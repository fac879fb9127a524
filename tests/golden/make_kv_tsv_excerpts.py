"""Writes excerpts of the reference's committed KV dumps (data, not code) as TSV fixtures:
  kv_q8_0_v4_excerpt.tsv  - runs/kv_q8_0_v4.tsv: the header line and every line of positions 0 and 36
  kv_none_v4_excerpt.tsv  - runs/kv_none_v4.tsv: the header line and every line of position 0
Both dumps were written by kv_dump (runtime_vk/bonsai_forward.h:1404-1488); the tests rebuild the
same arena bytes from kv_dump_v4.npz and check that bonsai_vk_amd.kvdump prints these lines exactly.
Run in the build container (the reference tree is not on the GPU box):
    python tests/golden/make_kv_tsv_excerpts.py
"""
import os

REF = "/root/reference"
HERE = os.path.dirname(os.path.abspath(__file__))


def excerpt(src, dst, positions):
    with open(os.path.join(REF, "runs", src)) as f, open(os.path.join(HERE, dst), "w") as g:
        for i, line in enumerate(f):
            if i == 0 or int(line.split()[1]) in positions:
                g.write(line)


if __name__ == "__main__":
    excerpt("kv_q8_0_v4.tsv", "kv_q8_0_v4_excerpt.tsv", {0, 36})
    excerpt("kv_none_v4.tsv", "kv_none_v4_excerpt.tsv", {0})
