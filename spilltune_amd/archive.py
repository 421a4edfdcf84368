"""On-disk quantized base archives (``nf4-g128``, ``int4-sym-g128``) in the
reference's ``rvft.quantized_base.v1`` layout, and direct-to-pinned loading of
whole layer images from them.

Layout (quantization/storage.py:15-72,186-221 of the reference, paths relative
to /root/reference/src/ram_vram_finetune): a directory holding one
``tensor-NNNNN.safetensors`` per checkpoint key (``payload`` uint8 +
``scales`` fp32 for a 4-bit matrix, ``value`` for a raw tensor), the allowed
tokenizer/config sidecars, ``rvft_quantization.json`` (format, family,
quantization, source/storage identities, per-key entries, per-file sha256)
and ``COMPLETE`` (sha256 of the marker).  The identities hash the same bytes
in the same order as storage.py:27-30,95-97,148-151,158-163, so an archive
written here and one written by the reference for the same source and format
carry the same identities.

What this build adds is the load side for the slot session: ``ArchiveReader``
checks every file's digest while it reads, and ``image_loader`` streams each
4-bit payload/scale and raw norm vector straight from its file into the
block's pinned slot image (``readinto`` on the pinned buffer; no intermediate
host tensor), which ``slots.Q4SlotSession`` then copies to the device in one
``hipMemcpyAsync`` per layer.
"""
from __future__ import annotations

import hashlib
import json
import math
import os
import shutil
import struct
import tempfile
from pathlib import Path

import torch
from safetensors import safe_open
from safetensors.torch import load_file, save_file

from . import codecs
from .codecs import GROUP, STRIDE, Record

MARKER = "rvft_quantization.json"
FORMAT = "rvft.quantized_base.v1"
# sidecar files an archive may carry next to its tensors (storage.py:16-17)
SIDECARS = frozenset({"config.json", "tokenizer.json", "tokenizer_config.json",
                      "special_tokens_map.json", "chat_template.jinja", "vocab.json", "merges.txt",
                      "added_tokens.json", "LICENSE", "LICENSE.txt", "LICENSE.md", "NOTICE",
                      "README.md"})
RAW_DTYPES = {"bfloat16": torch.bfloat16, "float32": torch.float32}
_ST_DTYPES = {"U8": (torch.uint8, 1), "F32": (torch.float32, 4), "BF16": (torch.bfloat16, 2)}
_READ_CHUNK = 1 << 22


# ----------------------------------------------------------------- hashing
def file_hash(path) -> str:
    h = hashlib.sha256()
    with Path(path).open("rb") as f:
        while chunk := f.read(1 << 20):
            h.update(chunk)
    return h.hexdigest()


def hash_tensor(h, name: str, tensor: torch.Tensor) -> None:
    """Name, dtype, shape, then the raw bytes (the identity convention of
    storage.py:27-30)."""
    h.update(name.encode())
    h.update(str(tensor.dtype).encode())
    h.update(str(tuple(tensor.shape)).encode())
    flat = tensor.detach().contiguous().view(torch.uint8).reshape(-1)
    for start in range(0, flat.numel(), 4 << 20):
        h.update(memoryview(flat[start:start + (4 << 20)].numpy()))


def encoded_size(shape, source_dtype: str, mode: str, *, selected: bool,
                 raw_dtype=torch.bfloat16) -> int:
    """Stored bytes of one entry (codecs.py:46-52 for the 4-bit formats)."""
    count = math.prod(shape)
    if mode != "none" and selected:
        return (count + GROUP - 1) // GROUP * (STRIDE + 4)
    if mode != "none":
        return count * torch.empty((), dtype=raw_dtype).element_size()
    return count * (4 if source_dtype == "F32" else 2)


# ---------------------------------------------------------- safetensors I/O
def safetensors_header(path) -> tuple[dict, int]:
    """(tensor name -> {dtype, shape, data_offsets}, byte offset of the data)."""
    with Path(path).open("rb") as f:
        raw = f.read(8)
        if len(raw) != 8:
            raise ValueError("truncated safetensors file")
        (n,) = struct.unpack("<Q", raw)
        if n > 100 << 20:
            raise ValueError("implausible safetensors header")
        header = json.loads(f.read(n))
    header.pop("__metadata__", None)
    return header, 8 + n


def inspect_checkpoint(path, family: str) -> dict:
    """Minimal report of a dense Llama-style safetensors checkpoint, with the
    fields ``export_quantized`` reads (the subset of the adapter inspection
    report of adapters/dense.py:40-112 that storage needs): ``text_config``,
    ``entries`` (file, shape, dtype), ``required`` (sorted keys),
    ``quantization_matrix_keys`` (decoder-layer 2-D matrices of >= 128
    elements), ``quantization_fp32_keys`` and ``quantized_export``."""
    root = Path(path)
    raw = json.loads((root / "config.json").read_text(encoding="utf-8"))
    if raw.get("model_type") != family:
        raise ValueError(f"unsupported_architecture: expected {family}")
    entries = {}
    for shard in sorted(root.glob("*.safetensors")):
        header, _ = safetensors_header(shard)
        for key, info in header.items():
            if key in entries:
                raise ValueError("duplicate checkpoint tensor")
            entries[key] = {"file": str(shard), "shape": list(info["shape"]),
                            "dtype": info["dtype"]}
    if not entries:
        raise ValueError("no safetensors tensors found")
    dtypes = {e["dtype"] for e in entries.values()}
    if not dtypes <= {"F32", "BF16"}:
        raise ValueError("unsupported_capability: FP32 or BF16 checkpoint required")
    return {"text_config": raw, "entries": entries, "required": sorted(entries),
            "quantization_matrix_keys": [k for k, e in entries.items()
                                         if k.startswith("model.layers.") and len(e["shape"]) == 2
                                         and math.prod(e["shape"]) >= GROUP],
            "quantization_fp32_keys": [],
            "quantized_export": {"version": 1, "formats": list(codecs.FORMATS),
                                 "rejection_reason": ""}}


def _require_export_capability(report: dict, mode: str) -> None:
    """Explicit per-adapter permission, as storage.py:172-183."""
    codecs.check_format(mode)
    cap = report.get("quantized_export")
    if not isinstance(cap, dict) or set(cap) != {"version", "formats", "rejection_reason"} \
            or cap["version"] != 1 or not isinstance(cap["formats"], list):
        raise ValueError("unsupported_quantization: missing or malformed adapter export capability")
    if mode not in cap["formats"]:
        raise ValueError("unsupported_quantization: "
                         + (cap["rejection_reason"] or "adapter did not validate this export format"))


def _encode_entry(value: torch.Tensor, mode: str, selected: bool, raw_dtype) -> Record:
    if selected:
        return codecs.encode(value, mode)
    out = value.to(raw_dtype).contiguous()
    for start in range(0, out.numel(), 32768):
        if not torch.isfinite(out.reshape(-1)[start:start + 32768]).all():
            raise ValueError("nonfinite raw weight")
    spec = {"version": 1, "shape": list(value.shape), "dtype": str(raw_dtype).split(".")[-1],
            "codec": "raw"}
    return Record(spec, {"value": out})


# --------------------------------------------------------------- export
def export_quantized(path, output, family: str, mode: str, *, report: dict | None = None) -> dict:
    """Write a quantized archive of the checkpoint at ``path`` (storage.py:186-221):
    one source tensor in memory at a time, staged in a temporary sibling
    directory and renamed into place when complete."""
    codecs.check_format(mode)
    path, output = Path(path), Path(output)
    if (path / MARKER).exists():
        raise ValueError("quantized re-encoding is not supported")
    report = report if report is not None else inspect_checkpoint(path, family)
    _require_export_capability(report, mode)
    output.parent.mkdir(parents=True, exist_ok=True)
    if output.exists():
        raise FileExistsError(output)
    matrices = set(report["quantization_matrix_keys"])
    fp32 = set(report["quantization_fp32_keys"])
    text = report["text_config"]
    source = hashlib.sha256(json.dumps(text, sort_keys=True).encode())
    stored = hashlib.sha256(json.dumps({"format": mode, "version": 1, "compute": "bf16",
                                        "config": text}, sort_keys=True).encode())
    temp = Path(tempfile.mkdtemp(prefix=".quant-stage-", dir=output.parent))
    try:
        entries, stored_bytes, quantized, max_src = {}, 0, 0, 0
        for index, key in enumerate(report["required"]):
            info = report["entries"][key]
            with safe_open(info["file"], framework="pt", device="cpu") as handle:
                value = handle.get_tensor(key).detach().contiguous()
            max_src = max(max_src, value.numel() * value.element_size())
            hash_tensor(source, key, value)
            raw_dtype = torch.float32 if key in fp32 else torch.bfloat16
            record = _encode_entry(value, mode, key in matrices, raw_dtype)
            del value
            name = f"tensor-{index:05d}.safetensors"
            save_file(record.parts, str(temp / name))
            stored.update(key.encode())
            stored.update(json.dumps(record.spec, sort_keys=True).encode())
            nbytes = 0
            for part, tensor in sorted(record.parts.items()):
                hash_tensor(stored, part, tensor)
                nbytes += tensor.numel() * tensor.element_size()
            stored_bytes += nbytes
            quantized += record.spec["codec"] != "raw"
            entries[key] = {"file": name, "shape": info["shape"], "dtype": info["dtype"],
                            "spec": record.spec, "stored_bytes": nbytes}
            del record
        if quantized < 1:
            raise ValueError("unsupported_quantization: no eligible decoder matrices")
        for name in sorted(SIDECARS):
            src = path / name
            if src.is_file():
                if src.is_symlink():
                    raise ValueError("symlink tokenizer/config export rejected")
                shutil.copyfile(src, temp / name)
        files = {p.name: file_hash(p) for p in sorted(temp.iterdir())}
        source_id, storage_id = source.hexdigest(), stored.hexdigest()
        meta = {"format": FORMAT, "family": family, "quantization": mode,
                "source_identity": source_id, "storage_identity": storage_id,
                "entries": entries, "files": files}
        (temp / MARKER).write_text(json.dumps(meta, sort_keys=True) + "\n", encoding="utf-8",
                                   newline="\n")
        (temp / "COMPLETE").write_text(file_hash(temp / MARKER) + "\n", encoding="utf-8",
                                       newline="\n")
        os.rename(temp, output)
        temp = None
        return {"output": str(output), "quantization": mode, "source_identity": source_id,
                "storage_identity": storage_id, "stored_bytes": stored_bytes,
                "max_source_tensor_bytes": max_src, "full_bf16_decoder_materialized": False,
                "quantized_matrices": quantized}
    finally:
        if temp is not None:
            shutil.rmtree(temp)


# ---------------------------------------------------------------- read side
def archive_entries(root, family: str, *, verify_files: bool = True) -> dict | None:
    """Validate an archive's marker, manifest, file digests, entry schema and
    tensor headers before any payload is read (storage.py:33-72).  Returns
    key -> entry (with ``file`` made absolute), or None when ``root`` is not an
    archive.  ``verify_files=False`` defers the per-file digests to
    ``ArchiveReader``, which checks them while it reads."""
    root = Path(root)
    marker = root / MARKER
    if not marker.exists():
        return None
    meta = json.loads(marker.read_text(encoding="utf-8"))
    if set(meta) != {"format", "family", "quantization", "source_identity", "storage_identity",
                     "entries", "files"} or meta["format"] != FORMAT or meta["family"] != family:
        raise ValueError("unsupported_quantization: archive schema/family")
    mode = meta["quantization"]
    codecs.check_format(mode)
    if not isinstance(meta["entries"], dict) or not meta["entries"]:
        raise ValueError("empty quantized archive")
    if (root / "COMPLETE").read_text(encoding="utf-8") != file_hash(marker) + "\n":
        raise ValueError("quantized archive manifest mismatch")
    files = meta["files"]
    if "config.json" not in files:
        raise ValueError("missing bound model configuration")
    for name, digest in files.items():
        if Path(name).name != name or (name not in SIDECARS and not (
                name.startswith("tensor-") and name.endswith(".safetensors"))) \
                or not (root / name).is_file() \
                or (verify_files and file_hash(root / name) != digest):
            raise ValueError("quantized archive file/hash mismatch")
    entries, used = {}, set()
    for key, entry in meta["entries"].items():
        if set(entry) != {"file", "shape", "dtype", "spec", "stored_bytes"} \
                or entry["file"] in used or entry["file"] not in files:
            raise ValueError("duplicate/missing quantized tensor file")
        used.add(entry["file"])
        spec, shape = entry["spec"], entry["shape"]
        if not isinstance(shape, list) or not shape or any(type(n) is not int or n < 1 for n in shape) \
                or entry["dtype"] not in {"F32", "BF16"}:
            raise ValueError("invalid logical tensor schema")
        if spec.get("shape") != shape or spec.get("codec") not in {"raw", mode}:
            raise ValueError("quantized logical shape/codec mismatch")
        selected = spec["codec"] != "raw"
        count = math.prod(shape)
        if spec.get("version") != 1 or spec.get("dtype") not in RAW_DTYPES:
            raise ValueError("invalid quantized archive policy/version/dtype")
        fields = {"version", "shape", "dtype", "codec"} | ({"group_size", "numel"} if selected else set())
        if set(spec) != fields or (selected and (spec["group_size"] != GROUP or spec["numel"] != count)):
            raise ValueError("invalid quantized archive group/numel")
        expected_bytes = encoded_size(shape, entry["dtype"], mode, selected=selected,
                                      raw_dtype=RAW_DTYPES[spec["dtype"]])
        if type(entry["stored_bytes"]) is not int or entry["stored_bytes"] != expected_bytes:
            raise ValueError("invalid stored byte budget")
        header, _ = safetensors_header(root / entry["file"])
        got = {k: (v["shape"], v["dtype"]) for k, v in header.items()}
        groups = (count + GROUP - 1) // GROUP
        want = ({"value": (shape, "BF16" if spec["dtype"] == "bfloat16" else "F32")} if not selected
                else {"payload": ([groups * STRIDE], "U8"), "scales": ([groups], "F32")})
        if got != want:
            raise ValueError("quantized archive tensor headers mismatch")
        entries[key] = {**entry, "file": str(root / entry["file"])}
    return entries


class ArchiveReader:
    """Reads records from a validated archive (the archive branch of
    ``WeightLoader``, storage.py:89-163).  Each tensor file is hashed as it is
    read and checked against the manifest.  Entries may be read in any order
    (layer images load block by block); ``finish()`` recomputes the storage
    identity over all records in key order -- from the buffers they were read
    into -- and returns the base identity
    ``sha256(source_identity + storage_identity)``."""

    def __init__(self, root, family: str, mode: str):
        codecs.check_format(mode)
        self.root = Path(root)
        self.entries = archive_entries(self.root, family, verify_files=False)
        if self.entries is None:
            raise ValueError("not a quantized archive")
        self.meta = json.loads((self.root / MARKER).read_text(encoding="utf-8"))
        if mode != self.meta["quantization"]:
            raise ValueError("unsupported_quantization: explicitly select archive format")
        self.mode = mode
        self.records = {}
        self.stored_bytes = 0

    def _config(self):
        return json.loads((self.root / "config.json").read_text(encoding="utf-8"))

    def _check_digest(self, file: Path, data_hash: str) -> None:
        if self.meta["files"].get(file.name) != data_hash:
            raise ValueError("quantized archive file/hash mismatch")

    def _account(self, key: str, record: Record) -> None:
        if key in self.records:
            raise ValueError(f"archive entry {key} read twice")
        self.records[key] = record
        self.stored_bytes += sum(t.numel() * t.element_size() for t in record.parts.values())

    def read(self, key: str) -> Record:
        """One entry as CPU tensors, digest-checked and schema-validated."""
        entry = self.entries[key]
        file = Path(entry["file"])
        self._check_digest(file, file_hash(file))
        record = Record(entry["spec"], load_file(str(file)))
        if record.spec["codec"] != "raw":
            codecs.validate_spec(record.spec, record.parts)
        self._account(key, record)
        return record

    def read_into(self, key: str, targets: dict) -> Record:
        """Stream entry ``key`` straight into caller-owned host buffers:
        ``targets`` maps part name -> a contiguous uint8 CPU tensor (pinned
        or not) of exactly that part's byte size.  The file is read once, in
        order, hashing as it goes; returns the record viewing those buffers."""
        entry = self.entries[key]
        file = Path(entry["file"])
        header, data0 = safetensors_header(file)
        if set(targets) != set(header):
            raise ValueError("read_into: parts do not match the archive entry")
        spans = sorted((info["data_offsets"][0], info["data_offsets"][1], part)
                       for part, info in header.items())
        h = hashlib.sha256()
        with file.open("rb") as f:
            h.update(f.read(data0))
            pos = 0
            for begin, end, part in spans:
                if begin != pos:
                    raise ValueError("safetensors data not contiguous")
                out = targets[part]
                if out.dtype != torch.uint8 or not out.is_contiguous() \
                        or out.numel() != end - begin or out.device.type != "cpu":
                    raise ValueError("read_into: target must be a contiguous uint8 host view "
                                     "of the part's size")
                view = memoryview(out.numpy())
                done = 0
                while done < end - begin:
                    got = f.readinto(view[done:min(done + _READ_CHUNK, end - begin)])
                    if not got:
                        raise ValueError("truncated archive tensor file")
                    h.update(view[done:done + got])
                    done += got
                pos = end
            rest = f.read()
            h.update(rest)
        self._check_digest(file, h.hexdigest())
        parts = {}
        for part, info in header.items():
            dtype, _ = _ST_DTYPES[info["dtype"]]
            parts[part] = targets[part].view(dtype).view(info["shape"])
        record = Record(entry["spec"], parts)
        if record.spec["codec"] != "raw":
            codecs.validate_spec(record.spec, record.parts)
        self._account(key, record)
        return record

    def finish(self) -> str:
        """Check that every entry was read and that the storage identity,
        hashed in key order over the records' buffers, matches the manifest
        (storage.py:155-163).  The buffers must still hold what was read."""
        if sorted(self.records) != sorted(self.entries):
            raise ValueError("archive loading order/inventory mismatch")
        stored = hashlib.sha256(json.dumps({"format": self.mode, "version": 1, "compute": "bf16",
                                            "config": self._config()}, sort_keys=True).encode())
        for key in sorted(self.records):
            record = self.records[key]
            stored.update(key.encode())
            stored.update(json.dumps(record.spec, sort_keys=True).encode())
            for part, tensor in sorted(record.parts.items()):
                hash_tensor(stored, part, tensor)
        storage = stored.hexdigest()
        if storage != self.meta["storage_identity"]:
            raise ValueError("quantized base identity mismatch")
        return hashlib.sha256((self.meta["source_identity"] + storage).encode()).hexdigest()

    # ------------------------------------------------- slot-image loading
    def block_specs(self, prefix: str) -> tuple[dict, dict]:
        """(storage_specs, raw entries) of the keys under ``prefix`` (e.g.
        ``model.layers.3.``), named without the prefix, in the form
        ``slots.plan_layout`` takes."""
        specs, raws = {}, {}
        for key, entry in self.entries.items():
            if not key.startswith(prefix):
                continue
            name = key[len(prefix):]
            if entry["spec"]["codec"] == "raw":
                raws[name] = entry
            else:
                specs[name] = {"spec": entry["spec"],
                               "parts": {"payload": f"@{name}/payload",
                                         "scales": f"@{name}/scales"}}
        return specs, raws

    def image_loader(self, prefix: str):
        """``fn(block, layout, out)`` filling a block's slot image ``out``
        (uint8, layout.nbytes) straight from the archive files: each 4-bit
        payload and scale vector and each raw tensor lands at its layout
        offset.  Use with ``slots.Q4SlotSession(image_loader=...)``."""
        def load(block, layout, out):
            out.zero_()
            for name in sorted(layout.entries):
                e = layout.entries[name]
                if e[0] == "q4":
                    _, _, _, po, pb, so, sb = e
                    self.read_into(prefix + name, {"payload": out[po:po + pb],
                                                   "scales": out[so:so + sb]})
                else:
                    _, _, _, o, nb = e
                    self.read_into(prefix + name, {"value": out[o:o + nb]})
        return load

    def block_host_weights(self, prefix: str) -> tuple[dict, dict]:
        """(host_weights, storage_specs) for a ``slots.BlockPlan`` of the layer
        under ``prefix`` whose image comes from ``image_loader``: raw entries
        appear as meta tensors (shape and dtype for the layout only)."""
        specs, raws = self.block_specs(prefix)
        host = {name: torch.empty(e["shape"], dtype=RAW_DTYPES[e["spec"]["dtype"]], device="meta")
                for name, e in raws.items()}
        return host, specs


__all__ = ["MARKER", "FORMAT", "SIDECARS", "file_hash", "hash_tensor", "encoded_size",
           "safetensors_header", "inspect_checkpoint", "export_quantized", "archive_entries",
           "ArchiveReader"]
