"""Tiny Llama-shaped safetensors checkpoint (config-1 sizes: hidden 256,
intermediate 688, 4 heads x 64) written the way a Hugging Face checkpoint
lies on disk, for the archive tests."""
import json

import torch
from safetensors.torch import save_file

BF = torch.bfloat16
CFG = {"model_type": "llama", "hidden_size": 256, "intermediate_size": 688,
       "num_hidden_layers": 2, "num_attention_heads": 4, "num_key_value_heads": 4,
       "head_dim": 64, "vocab_size": 1024, "rms_norm_eps": 1e-5, "hidden_act": "silu",
       "max_position_embeddings": 256, "tie_word_embeddings": False}
LAYER = {"self_attn.q_proj.weight": (256, 256), "self_attn.k_proj.weight": (256, 256),
         "self_attn.v_proj.weight": (256, 256), "self_attn.o_proj.weight": (256, 256),
         "mlp.gate_proj.weight": (688, 256), "mlp.up_proj.weight": (688, 256),
         "mlp.down_proj.weight": (256, 688), "input_layernorm.weight": (256,),
         "post_attention_layernorm.weight": (256,)}


def make_checkpoint(root, seed=1234, layers=2):
    root.mkdir(parents=True)
    g = torch.Generator().manual_seed(seed)
    tensors = {"model.embed_tokens.weight": torch.randn(1024, 256, generator=g).to(BF),
               "model.norm.weight": (1 + 0.05 * torch.randn(256, generator=g)).to(BF),
               "lm_head.weight": (0.02 * torch.randn(1024, 256, generator=g)).to(BF)}
    for i in range(layers):
        for name, shape in LAYER.items():
            t = (1 + 0.05 * torch.randn(shape, generator=g)) if len(shape) == 1 \
                else 0.02 * torch.randn(shape, generator=g)
            tensors[f"model.layers.{i}.{name}"] = t.to(BF)
    save_file(tensors, str(root / "model.safetensors"))
    (root / "config.json").write_text(json.dumps(CFG))
    (root / "secret.token").write_text("not copied")
    return tensors
