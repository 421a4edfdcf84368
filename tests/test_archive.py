"""On-disk quantized base archive (rvft.quantized_base.v1 layout): export,
validation, digest and identity checks, and direct filling of slot images.
Mirrors the reference's archive tests (tests/test_quantization.py:243-305:
round trip, corruption/format/shape rejection, explicit format selection)
on a config-1-shaped tiny Llama checkpoint; runs without a GPU."""
import hashlib
import json
import sys
from pathlib import Path

import pytest
import torch

from spilltune_amd import archive, codecs, slots

from _ckpt import LAYER, make_checkpoint


@pytest.fixture(params=list(codecs.FORMATS))
def exported(tmp_path, request):
    src = tmp_path / "source"
    tensors = make_checkpoint(src)
    out = tmp_path / "archive"
    info = archive.export_quantized(src, out, "llama", request.param)
    return request.param, tensors, out, info


def test_export_layout_and_round_trip(exported):
    mode, tensors, out, info = exported
    names = sorted(p.name for p in out.iterdir())
    assert "secret.token" not in names and "config.json" in names
    assert {archive.MARKER, "COMPLETE"} <= set(names)
    meta = json.loads((out / archive.MARKER).read_text())
    assert meta["format"] == "rvft.quantized_base.v1" and meta["quantization"] == mode
    entries = archive.archive_entries(out, "llama")
    assert set(entries) == set(tensors)
    assert info["quantized_matrices"] == 14 and not info["full_bf16_decoder_materialized"]
    reader = archive.ArchiveReader(out, "llama", mode)
    for key in sorted(tensors):
        rec = reader.read(key)
        src = tensors[key]
        if key.startswith("model.layers.") and src.dim() == 2:
            want = codecs.encode(src, mode)
            assert rec.spec == want.spec
            assert torch.equal(rec.parts["payload"], want.parts["payload"])
            assert torch.equal(rec.parts["scales"], want.parts["scales"])
            assert entries[key]["stored_bytes"] == src.numel() // 128 * 68
        else:
            assert rec.spec == {"version": 1, "shape": list(src.shape), "dtype": "bfloat16",
                                "codec": "raw"}
            assert torch.equal(rec.parts["value"], src)
    identity = reader.finish()
    assert identity == hashlib.sha256(
        (info["source_identity"] + info["storage_identity"]).encode()).hexdigest()


def test_identity_tracks_source_and_storage(tmp_path):
    """The storage identity hashes the stored parts: a different format or a
    different tensor changes it; the same source re-exported reproduces it."""
    src = tmp_path / "source"
    make_checkpoint(src)
    a = archive.export_quantized(src, tmp_path / "a", "llama", "nf4-g128")
    b = archive.export_quantized(src, tmp_path / "b", "llama", "nf4-g128")
    c = archive.export_quantized(src, tmp_path / "c", "llama", "int4-sym-g128")
    assert a["storage_identity"] == b["storage_identity"] != c["storage_identity"]
    assert a["source_identity"] == b["source_identity"] == c["source_identity"]
    src2 = tmp_path / "source2"
    make_checkpoint(src2, seed=99)
    d = archive.export_quantized(src2, tmp_path / "d", "llama", "nf4-g128")
    assert d["source_identity"] != a["source_identity"]
    assert d["storage_identity"] != a["storage_identity"]


def test_identities_match_the_reference_loader(tmp_path):
    """Source, storage and base identities of an int4-sym-g128 export equal the
    ones the reference's own loader computed for the same synthetic checkpoint
    (quantization/storage.py:89-165; tests/golden/archive_identity.json,
    written by tests/golden/make_archive_identity.py), and reading the archive
    back reproduces the base identity from the stored bytes."""
    sys.path.insert(0, str(Path(__file__).resolve().parent / "golden"))
    import make_archive_identity as gold

    golden = json.loads(gold.FIXTURE.read_text())
    report = gold.checkpoint(tmp_path / "src")
    # the bound configuration the reader hashes is the exported text config
    (tmp_path / "src" / "config.json").write_text(json.dumps(report["text_config"]))
    info = archive.export_quantized(tmp_path / "src", tmp_path / "out", "llama", gold.MODE,
                                    report=report)
    assert info["source_identity"] == golden["source_identity"]
    assert info["storage_identity"] == golden["storage_identity"]
    assert info["stored_bytes"] == golden["stored_bytes"]
    assert info["quantized_matrices"] == golden["quantized_tensors"]
    reader = archive.ArchiveReader(tmp_path / "out", "llama", gold.MODE)
    for key in report["required"]:
        reader.read(key)
    assert reader.finish() == golden["identity"]


def test_image_loader_fills_the_packed_layout_in_any_order(exported):
    """Slot images streamed from the archive files equal the images packed
    from freshly encoded host tensors; layers may load in any order and the
    storage identity still verifies."""
    mode, tensors, out, _ = exported
    reader = archive.ArchiveReader(out, "llama", mode)
    for index in (1, 0):
        prefix = f"model.layers.{index}."
        block = slots.make_archive_block(reader, index, heads=4, kv_heads=4, head_dim=64, eps=1e-5,
                                         rank=8, alpha=16.0, targets=("self_attn.q_proj",),
                                         device="cpu")
        layout = slots.plan_layout(block)
        img = torch.empty(layout.nbytes, dtype=torch.uint8)
        reader.image_loader(prefix)(block, layout, img)
        weights = {n: tensors[prefix + n] for n in LAYER}
        ref_block = slots.make_dense_block(index, weights, codec=mode, heads=4, kv_heads=4,
                                           head_dim=64, eps=1e-5, rank=8, alpha=16.0,
                                           targets=("self_attn.q_proj",), device="cpu")
        ref_layout = slots.plan_layout(ref_block)
        assert ref_layout.entries == layout.entries and ref_layout.nbytes == layout.nbytes
        ref_img = torch.empty(ref_layout.nbytes, dtype=torch.uint8)
        slots.pack_image(ref_block, ref_layout, ref_img)
        assert torch.equal(img, ref_img)
    for key in sorted(tensors):
        if not key.startswith("model.layers."):
            reader.read(key)
    reader.finish()


def test_incomplete_or_tampered_reads_rejected(exported):
    mode, tensors, out, _ = exported
    reader = archive.ArchiveReader(out, "llama", mode)
    reader.read("model.norm.weight")
    with pytest.raises(ValueError, match="order/inventory"):
        reader.finish()
    with pytest.raises(ValueError, match="read twice"):
        reader.read("model.norm.weight")
    # a flipped payload byte: the digest check on read catches it
    meta = json.loads((out / archive.MARKER).read_text())
    key = "model.layers.0.mlp.up_proj.weight"
    f = out / meta["entries"][key]["file"]
    data = bytearray(f.read_bytes())
    data[-1] ^= 1
    f.write_bytes(bytes(data))
    with pytest.raises(ValueError, match="hash mismatch"):
        archive.ArchiveReader(out, "llama", mode).read(key)
    with pytest.raises(ValueError, match="hash mismatch"):
        archive.archive_entries(out, "llama")


def test_corruption_format_and_family_rejected(tmp_path):
    src = tmp_path / "source"
    make_checkpoint(src, layers=1)
    out = tmp_path / "q"
    archive.export_quantized(src, out, "llama", "nf4-g128")
    with pytest.raises(ValueError, match="explicitly select"):
        archive.ArchiveReader(out, "llama", "int4-sym-g128")
    with pytest.raises(ValueError, match="schema/family"):
        archive.archive_entries(out, "qwen2")
    for mode in ("nf4", "Q6_K", "Q8_0", "FP8"):
        with pytest.raises(ValueError, match="unsupported_quantization"):
            archive.export_quantized(src, tmp_path / mode, "llama", mode)
    with pytest.raises(FileExistsError):
        archive.export_quantized(src, out, "llama", "nf4-g128")
    with pytest.raises(ValueError, match="re-encoding"):
        archive.export_quantized(out, tmp_path / "again", "llama", "nf4-g128")
    # appended bytes (the reference's corruption case), then a tampered manifest
    meta = json.loads((out / archive.MARKER).read_text())
    f = out / next(n for n in meta["files"] if n.startswith("tensor-"))
    f.write_bytes(f.read_bytes() + b"x")
    with pytest.raises(ValueError, match="hash mismatch"):
        archive.archive_entries(out, "llama")
    (out / archive.MARKER).write_text(json.dumps(meta) + " ")
    with pytest.raises(ValueError, match="manifest mismatch"):
        archive.archive_entries(out, "llama")


def test_entry_schema_checks(tmp_path):
    src = tmp_path / "source"
    make_checkpoint(src, layers=1)
    out = tmp_path / "q"
    archive.export_quantized(src, out, "llama", "int4-sym-g128")

    def rewrite(mutate):
        meta = json.loads((out / archive.MARKER).read_text())
        mutate(meta)
        (out / archive.MARKER).write_text(json.dumps(meta, sort_keys=True) + "\n")
        (out / "COMPLETE").write_text(archive.file_hash(out / archive.MARKER) + "\n")

    key = "model.layers.0.self_attn.q_proj.weight"
    rewrite(lambda m: m["entries"][key].update(stored_bytes=1))
    with pytest.raises(ValueError, match="stored byte budget"):
        archive.archive_entries(out, "llama")
    rewrite(lambda m: m["entries"][key].update(stored_bytes=256 * 256 // 128 * 68,
                                               shape=[128, 512]))
    with pytest.raises(ValueError, match="shape/codec mismatch"):
        archive.archive_entries(out, "llama")


def test_export_capability_is_explicit(tmp_path):
    src = tmp_path / "source"
    make_checkpoint(src, layers=1)
    report = archive.inspect_checkpoint(src, "llama")
    report["quantized_export"] = {"version": 1, "formats": ["int4-sym-g128"],
                                  "rejection_reason": "nf4 not validated for this adapter"}
    with pytest.raises(ValueError, match="nf4 not validated"):
        archive.export_quantized(src, tmp_path / "q", "llama", "nf4-g128", report=report)
    del report["quantized_export"]
    with pytest.raises(ValueError, match="malformed"):
        archive.export_quantized(src, tmp_path / "q", "llama", "nf4-g128", report=report)


def test_read_into_streams_into_caller_buffers(exported):
    mode, tensors, out, _ = exported
    reader = archive.ArchiveReader(out, "llama", mode)
    key = "model.layers.1.mlp.down_proj.weight"
    groups = tensors[key].numel() // 128
    pay = torch.empty(groups * 64, dtype=torch.uint8)
    sc = torch.empty(groups * 4, dtype=torch.uint8)
    rec = reader.read_into(key, {"payload": pay, "scales": sc})
    want = codecs.encode(tensors[key], mode)
    assert rec.parts["payload"].data_ptr() == pay.data_ptr()
    assert torch.equal(pay, want.parts["payload"])
    assert torch.equal(sc.view(torch.float32), want.parts["scales"])
    with pytest.raises(ValueError, match="size"):
        reader.read_into("model.layers.1.mlp.up_proj.weight",
                         {"payload": torch.empty(3, dtype=torch.uint8),
                          "scales": torch.empty(3, dtype=torch.uint8)})
