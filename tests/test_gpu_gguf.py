"""Loading a model from its GGUF file (cpv_model_load_gguf) on the GPU.

A seeded random-init qwen35 file is written, loaded by the library and run;
the oracle gets the same tensor bytes.  The round (logits, hidden, preds, the
MTP chain) must be bit-identical, so the file path loses nothing against
handing over the tensors one by one.
"""
import numpy as np
import pytest

from oracle import cpvo

from codpiece_amd import gguf

pytestmark = pytest.mark.gpu

K = dict(n_layer=2, n_embd=512, n_head=8, n_head_kv=2, head_dim=64, n_ff=1536, n_vocab=4096, n_rot=64,
         rope_sections=(11, 11, 10, 0), rms_eps=1e-6, freq_base=1e6)


@pytest.mark.parametrize("qtype,head_type", [(gguf.Q4_K, gguf.Q6_K), (gguf.Q8_0, gguf.Q8_0)])
def test_file_model_round_equals_oracle(tmp_path, qtype, head_type):
    from codpiece_amd.model import Model, Session
    from codpiece_amd.runtime import Context
    p = tmp_path / "m.gguf"
    tensors = gguf.write_seeded_model(p, seed=5, qtype=qtype, head_type=head_type, **K)
    ctx = Context(0)
    print("load", p.stat().st_size, "bytes", flush=True)
    gm = Model.from_gguf(ctx, p)
    om = cpvo.Model(dict(K, rope_sections=list(K["rope_sections"]), has_mtp=1))
    for name, (t, dims, data) in tensors.items():
        om.set_tensor(name, t, data, dims[0], dims[1])
    rng = np.random.default_rng(6)
    prompt = rng.integers(0, K["n_vocab"], size=50).tolist()
    g, o = Session(gm, 256), cpvo.Session(om, 256)
    g.prefill(prompt[:45])
    o.prefill(prompt[:45])
    a = g.step_fused_cached(prompt[45:], 4, want_logits=True)
    b = o.step_fused_cached(prompt[45:], 4, want_logits=True)
    assert np.array_equal(a.logits.cpu().numpy().view(np.uint32), b[3].view(np.uint32))
    assert np.array_equal(a.hidden.cpu().numpy().view(np.uint32), b[4].view(np.uint32))
    assert a.preds == b[0].tolist() and a.chain == b[1].tolist()
    g.free()
    o.free()
    gm.free()
    om.free()
    ctx.close()


def test_file_the_model_cannot_take_is_refused(tmp_path):
    from codpiece_amd import _lib
    from codpiece_amd.model import Model
    from codpiece_amd.runtime import Context
    ctx = Context(0)
    p = tmp_path / "bad.gguf"
    w = gguf.Writer()
    w.add_str("general.architecture", "qwen35")
    for k, v in {"qwen35.block_count": 2, "qwen35.embedding_length": 256, "qwen35.attention.head_count": 4,
                 "qwen35.attention.head_count_kv": 2, "qwen35.feed_forward_length": 512}.items():
        w.add_u32(k, v)
    w.add_str_array("tokenizer.ggml.tokens", ["a"] * 8)
    w.write(p)                      # full_attention_interval defaults to 4: recurrent layers
    with pytest.raises(_lib.CpvError) as e:
        Model.from_gguf(ctx, p)
    assert e.value.status == _lib.CPV_EUNSUPPORTED
    # a tensor the model does not know
    p2 = tmp_path / "extra.gguf"
    t = gguf.seeded_tensors(1, 256, 4, 2, 64, 512, 64, has_mtp=False)
    w = gguf.Writer()
    w.add_str("general.architecture", "qwen35")
    for k, v in {"qwen35.block_count": 1, "qwen35.embedding_length": 256, "qwen35.attention.head_count": 4,
                 "qwen35.attention.head_count_kv": 2, "qwen35.feed_forward_length": 512,
                 "qwen35.full_attention_interval": 1}.items():
        w.add_u32(k, v)
    w.add_str_array("tokenizer.ggml.tokens", ["a"] * 64)
    for name, (gt, dims, data) in t.items():
        w.add_tensor(name, gt, dims, data)
    w.add_tensor("blk.0.ssm_conv1d.weight", gguf.F32, [4, 1], np.zeros(4, np.float32))
    w.write(p2)
    with pytest.raises(_lib.CpvError) as e:
        Model.from_gguf(ctx, p2)
    assert "ssm_conv1d" in str(e.value)
    ctx.close()
