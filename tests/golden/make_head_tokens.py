"""Writes tests/golden/head_tokens_65536.npy: the reference's own trimmed-head token set (65536 ascending ids,
qwen/head_tokens_65536.npy in the reference repository, the head of its Qwen2.5-Coder-0.5B build), kept as a
fixture so the GPU tests can build a Qwen2-0.5B-shape model with a realistic head.  The array is read with
numpy's pickle-free loader and written back unchanged.

    python tests/golden/make_head_tokens.py [/root/reference]"""
import os
import sys

import numpy as np

ref = sys.argv[1] if len(sys.argv) > 1 else "/root/reference"
ids = np.load(os.path.join(ref, "qwen", "head_tokens_65536.npy"), allow_pickle=False)
assert ids.dtype == np.int32 and ids.shape == (65536,) and (np.diff(ids) > 0).all()
np.save(os.path.join(os.path.dirname(os.path.abspath(__file__)), "head_tokens_65536.npy"), ids)
print(f"{len(ids)} ids, {ids[0]} .. {ids[-1]}")
