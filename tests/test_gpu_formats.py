"""Weight files made by the format tooling, and the reference's own head token set, through the device loop
(MI355X), in the strict mode against the reference's own qwen.c (oracle/_ref/libref_qwen.so): bit for bit.

  - GGUF -> .qwb (formats/qwb.py from_gguf, the role of tools/gguf2qwb.py:36-61, 90-107): a GGUF holding the
    tensors of a synthetic Qwen2-0.5B-shape model is converted back to .qwb, validated (formats/qwb.py check,
    the role of tools/qwb_check.py:19-62) and decoded;
  - a Qwen2-0.5B-shape model (24 layers) whose trimmed head is the reference's own token set
    (qwen/head_tokens_65536.npy, kept as tests/golden/head_tokens_65536.npy by tests/golden/make_head_tokens.py),
    which holds the stop ids 151643 and 151645: greedy decoding may stop at them, on both sides alike."""
import os

import numpy as np
import pytest

from helpers import GOLDEN, pkg, synth
from test_formats import qwb, qwb_to_gguf
from test_gpu_strict import RefQwen, c3_prompt, check_bitwise

pytestmark = pytest.mark.gpu


def decode_both(path, ctx, prompt, n):
    ref = RefQwen(path, ctx)
    ids_r, lg_r = ref.generate(prompt, n)
    m = pkg().Model(path, ctx)
    m.set_strict(True)
    r = m.generate(prompt, n, logits=True)
    return m, ref, r, ids_r, lg_r


def test_gguf_converted_model_decodes_bitwise_like_the_reference(tmp_path):
    src = synth("qwb", str(tmp_path / "src.qwb"), "c3", 43, "layers=2")
    head = qwb_to_gguf(src, str(tmp_path / "m.gguf"))
    out = str(tmp_path / "conv.qwb")
    qwb.from_gguf(str(tmp_path / "m.gguf"), head, out)
    qwb.check(out, str(tmp_path / "m.gguf"))
    ctx = 16 + 48
    prompt = c3_prompt(head, 16, 44)
    m, ref, r, ids_r, lg_r = decode_both(out, ctx, prompt, 48)
    assert len(ids_r) == 48
    check_bitwise(m, ref, r["ids"], r["logits"], ids_r, lg_r, len(lg_r))
    m.close()
    # the converted file decodes exactly like the file its tensors came from
    m = pkg().Model(src, ctx)
    m.set_strict(True)
    r0 = m.generate(prompt, 48, logits=True)
    m.close()
    assert np.array_equal(r0["logits"], r["logits"]) and list(r0["ids"]) == list(r["ids"])


def test_c3_with_the_reference_head_token_set(tmp_path):
    ids = np.load(os.path.join(GOLDEN, "head_tokens_65536.npy"), allow_pickle=False)
    f = str(tmp_path / "head_ids.bin")
    ids.astype("<i4").tofile(f)
    p = synth("qwb", str(tmp_path / "c3h.qwb"), "c3", 45, f"head_ids={f}")
    ctx = 24 + 64
    prompt = c3_prompt(ids, 24, 46)
    m, ref, r, ids_r, lg_r = decode_both(p, ctx, prompt, 64)
    assert np.array_equal(ref.head_ids, ids) and np.array_equal(m.head_ids, ids)
    print(f"reference: {len(ids_r)} ids over {len(lg_r)} positions")
    check_bitwise(m, ref, r["ids"], r["logits"], ids_r, lg_r, len(lg_r))
    m.close()
