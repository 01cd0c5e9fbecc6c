"""A Qwen2 GGUF (tests/gguf_writer.py, the reference's tensor names) loaded into a decoder with
muyo_decoder_load_gguf: every tensor bit-identical to the oracle model the file was written from
(q, k and v stacked into ATTN_QKV), and greedy ids equal to the oracle's, with the LM head tied to
the embedding or a separate output.weight."""
import numpy as np
import pytest

import gguf_writer as gw
from conftest import close

pytestmark = pytest.mark.gpu

SHAPE = dict(layers=2, hidden=256, ffn=512, heads=4, kv_heads=2, head_dim=64, vocab=6000, max_seq=128)


@pytest.mark.parametrize("untied,order,alignment", [(False, "reference", 32), (True, "reversed", 64)])
def test_gguf_load_and_decode(tmp_path, mh, gpu, orc, untied, order, alignment):
    model = orc.Model(**SHAPE, untied_output=untied)
    model.fill_random(77)
    path = tmp_path / "model.gguf"
    gw.qwen2_file(path, model, alignment=alignment, order=order)
    with mh.Gguf(path) as g:
        cfg = g.qwen2_config(SHAPE["max_seq"])
        assert cfg.untiedOutput == int(untied)
        with mh.Decoder(cfg) as dec:
            dec.load_gguf(g)
            for (kind, layer), arr in model.t.items():
                if kind in ("KCACHE", "VCACHE"):
                    continue
                got = np.empty_like(arr)
                dec.download(kind, layer, got)
                assert np.array_equal(got, arr), (kind, layer)
            token, ids, want = 11, [], []
            for pos in range(12):
                got = dec.step(token, pos)
                best, logits, _ = model.step(token, pos)
                gpu_logits = np.empty(SHAPE["vocab"], np.float32)
                dec.download("LOGITS", 0, gpu_logits)
                assert close(gpu_logits, logits, 1e-3) == 0, pos
                ids.append(got)
                want.append(best)
                token = got
            assert ids == want


def test_gguf_refuses_a_different_decoder(tmp_path, mh, gpu, orc):
    model = orc.Model(**SHAPE)
    model.fill_random(3)
    path = tmp_path / "model.gguf"
    gw.qwen2_file(path, model)
    other = dict(SHAPE, ffn=768)
    with mh.Gguf(path) as g, mh.Decoder(mh.qwen2_config(**other)) as dec:
        with pytest.raises(mh.MuyoError) as e:
            dec.load_gguf(g)
        assert e.value.status == mh.MUYO_E_CONTRACT
