"""The adapter factory end to end on the GPU: a tiny Llama checkpoint
(benchmark config 1 shapes) exported to an nf4-g128 archive, built through
the reference's factory call, streamed through Q4SlotSession (the engine's
one-line session swap) and trained for 30 AdamW steps on two cycled rows
against the CPU oracle's loss curve (north-star criterion |d loss| <= 1e-2)."""
import hashlib
import math

import numpy as np
import pytest
import torch

from oracle import layer as OL
from spilltune_amd import adapter, archive, engine, slots

from _ckpt import make_checkpoint

pytestmark = pytest.mark.gpu
BF = torch.bfloat16


def _decoded_layer(block, img, oracle_codec):
    """bf16 weights of one layer from its packed slot image (oracle decode)."""
    out = {}
    for name, e in slots.plan_layout(block).entries.items():
        if e[0] == "q4":
            _, codec, shape, po, pb, so, sb = e
            payload = img[po:po + pb].numpy()
            scales = img[so:so + sb].view(torch.float32).numpy()
            bits = oracle_codec.decode4(payload, scales, math.prod(shape), lut=oracle_codec.NF4_LUT)
            out[name] = torch.from_numpy(bits.astype(np.int16)).view(BF).view(shape)
        else:
            _, dtype, shape, o, nb = e
            out[name] = img[o:o + nb].view(dtype).view(shape).clone()
    return out


def test_factory_trains_like_the_oracle(tmp_path, oracle_codec):
    src = tmp_path / "source"
    tensors = make_checkpoint(src)
    out = tmp_path / "archive"
    info = archive.export_quantized(src, out, "llama", "nf4-g128")
    factory = adapter.FACTORIES["llama_q4_hip_all_targets"]
    dev = torch.device("cuda:0")
    model = factory(str(out), rank=8, alpha=16.0, device="cuda:0", host_budget_bytes=1 << 30,
                    device_budget_bytes=1 << 30, quantization="nf4-g128", quantized_compute="bf16")
    assert model.identity == hashlib.sha256(
        (info["source_identity"] + info["storage_identity"]).encode()).hexdigest()
    assert len(model.blocks) == 2 and model.device == dev
    assert model.artifact_key(1, "self_attn.q_proj", "A") == \
        "base_model.model.model.layers.1.self_attn.q_proj.lora_A.weight"
    meta = model.runtime_metadata()
    assert meta["layer_count"] == 2 and meta["lora_targets"] == list(adapter.ALL_TARGETS)
    assert torch.equal(model.embedding, tensors["model.embed_tokens.weight"])
    # LoRA init as config 1: A ~ kaiming_uniform(a=sqrt(5)), B = 0
    g = torch.Generator().manual_seed(3)
    oracle_loras, oracle_layers = [], []
    for block in model.blocks:
        lo = {}
        for name in sorted(block.adapters):
            p = block.adapters[name]
            bound = 1.0 / math.sqrt(p.in_features)
            A = (torch.rand(p.A.shape, generator=g) * 2 - 1) * bound
            with torch.no_grad():
                p.A.copy_(A)
                p.B.zero_()
            lo[name] = OL.Lora(name, A, torch.zeros(p.B.shape), p.alpha)
        oracle_loras.append(lo)
        oracle_layers.append(_decoded_layer(block, block.host_image, oracle_codec))
    # the engine's session line, swapped: the adapter's pinned images are adopted
    session = slots.Q4SlotSession(model.blocks, dev, host_budget_bytes=1 << 30,
                                  device_budget_bytes=1 << 30)
    assert all(session.images[id(b)].data_ptr() == b.host_image.data_ptr() for b in model.blocks)
    gd = torch.Generator().manual_seed(7)
    rows = []
    for _ in range(2):
        ids = torch.randint(0, 1024, (2, 128), generator=gd)
        rows.append((ids, ids.clone()))
    steps, lr = 30, 1e-2
    gpu = engine.train(model, session, rows, steps=steps, lr=lr, token_chunk=64)
    cfg = dict(heads=4, kv_heads=4, head_dim=64, eps=1e-5)
    cpu = OL.train_reference(model.embedding, tensors["model.norm.weight"],
                             tensors["lm_head.weight"], oracle_layers, oracle_loras, rows, cfg=cfg,
                             theta=10000.0, steps=steps, lr=lr, token_chunk=64)
    diff = np.abs(np.array(gpu) - np.array(cpu))
    print(f"loss gpu {gpu[0]:.4f}->{gpu[-1]:.4f}, cpu {cpu[0]:.4f}->{cpu[-1]:.4f}, "
          f"max |diff| {diff.max():.2e}")
    assert gpu[-1] < gpu[0] - 1.0, "training did not reduce the loss"
    assert diff.max() <= 1e-2, (diff.max(), gpu, cpu)
    session.close()
    model.close()
