"""Adapter factory with the reference's registry signature (CPU side):
registration, the factory's keyword surface and argument rules, the
archive inspector and the config checks (adapters/registry.py:6-15,
training/engine.py:127-130, adapters/protocol.py:23-34, adapters/dense.py:
40-112,178-263 of /root/reference/src/ram_vram_finetune)."""
import inspect

import pytest

from spilltune_amd import adapter, archive

from _ckpt import CFG, make_checkpoint

REFERENCE_FACTORY_KWARGS = {"rank", "alpha", "device", "host_budget_bytes", "device_budget_bytes",
                            "quantization", "quantized_compute"}
PROTOCOL = ("blocks", "embedding", "head", "identity", "device")
PROTOCOL_METHODS = ("positions_and_masks", "terminal_norm", "artifact_key", "runtime_metadata",
                    "close")


def test_factory_signature_matches_the_engine_call():
    for name, factory in adapter.FACTORIES.items():
        sig = inspect.signature(factory)
        params = sig.parameters
        assert list(params)[0] == "path", name
        assert REFERENCE_FACTORY_KWARGS <= set(params), name
        for k in REFERENCE_FACTORY_KWARGS:
            assert params[k].kind == inspect.Parameter.KEYWORD_ONLY, (name, k)
    for meth in PROTOCOL_METHODS:
        assert callable(getattr(adapter.ArchiveDenseAdapter, meth))


def test_register_all_uses_distinct_names_and_the_inspector():
    seen = {}

    def register(name, factory, *, inspector=None):  # the reference's signature
        assert name not in seen and callable(factory) and callable(inspector)
        assert name not in {"qwen35", "llama", "qwen2", "qwen3", "qwen3_moe", "deepseek_v3",
                            "gpt_oss", "glm4_moe_lite", "qwen35_moe"}
        seen[name] = (factory, inspector)
    names = adapter.register_all(register)
    assert set(names) == set(seen) == set(adapter.FACTORIES)
    assert adapter.FACTORIES["llama_q4_hip"] is adapter.LlamaArchiveAdapter
    assert adapter.FACTORIES["llama_q4_hip_all_targets"].keywords["targets"] == adapter.ALL_TARGETS


def test_default_targets_are_the_references():
    assert adapter.REFERENCE_TARGETS == ("self_attn.q_proj", "self_attn.v_proj", "self_attn.o_proj")


@pytest.mark.parametrize("kw,err,msg", [
    ({"quantized_compute": "fp8"}, ValueError, "only storage plus BF16 compute"),
    ({"quantization": "none"}, ValueError, "explicit format required"),
    ({"quantization": "nf4"}, ValueError, "explicit format required"),
    ({"device": "cpu"}, ValueError, "runs on a GPU device"),
])
def test_factory_argument_rules(tmp_path, kw, err, msg):
    args = dict(rank=4, alpha=8.0, device="cuda:0", quantization="nf4-g128")
    args.update(kw)
    with pytest.raises(err, match=msg):
        adapter.LlamaArchiveAdapter(tmp_path, **args)


def test_inspector_and_config_rules(tmp_path):
    src = tmp_path / "source"
    make_checkpoint(src)
    out = tmp_path / "archive"
    info = archive.export_quantized(src, out, "llama", "nf4-g128")
    rep = adapter.inspect_archive(out)
    assert rep["quantization"] == "nf4-g128" and rep["family"] == "llama"
    assert rep["layers"] == CFG["num_hidden_layers"]
    assert rep["storage_identity"] == info["storage_identity"]
    cfg = adapter._text_config(dict(CFG), "llama")
    assert (cfg["heads"], cfg["kv_heads"], cfg["head_dim"], cfg["theta"]) == (4, 4, 64, 10000.0)
    for bad, msg in (({"model_type": "qwen3"}, "expected llama"),
                     ({"hidden_act": "gelu"}, "dropout/activation"),
                     ({"attention_bias": True}, "projection biases"),
                     ({"rope_parameters": {"rope_type": "yarn", "rope_theta": 1e4}}, "default full"),
                     ({"sliding_window": 128}, "sliding window"),
                     ({"tie_word_embeddings": True}, "tied embeddings")):
        with pytest.raises(ValueError, match=msg):
            adapter._text_config(dict(CFG, **bad), "llama")
