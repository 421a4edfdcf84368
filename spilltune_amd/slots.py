"""Packed 4-bit layer slots: pinned host arenas -> device slots on a copy stream.

Engine-visible surface of the reference's sessions (paths relative to
/root/reference/src/ram_vram_finetune): ``run()`` (serial, non-reentrant,
run-token scoped), ``reloader(block)`` returning a lease with
``borrow(phase)``, and the counters/trace ``engine.run`` reads
(memory.py:140-290, prefetch.py:47-252, engine.py:136-143,168-188,209-228).

What moves is the packed storage itself: each block is laid out once, at
construction, as ONE contiguous byte image (4-bit payloads, fp32 scales and
raw norm vectors, 256-byte aligned; q|k|v and gate|up payloads/scales packed
back to back so they can run as one GEMM) in a pinned host buffer.  A load is
one ``hipMemcpyAsync`` of that image into a device slot on a dedicated copy
stream (default priority) -- no decode pass: the GEMMs dequantise from the
slot.  Ordering follows prefetch.py:162-223: a ``ready`` event admits use on
the compute stream, a ``consumed`` event recorded after the whole consumer
scope (recompute, VJP and gradient accumulation) admits overwrite; the next
block in the phase direction is prefetched into the least recently used free
slot, and the last forward block is a backward cache hit.
"""
from __future__ import annotations

import threading
from contextlib import contextmanager
from dataclasses import dataclass, field
from typing import Any, Callable

import torch

from . import codecs
from .ops import Q4Weight

ALIGN = 256
# projections whose storage is packed back to back (row-concatenation groups)
FUSION_GROUPS = (("self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj"),
                 ("self_attn.q_a_proj", "self_attn.kv_a_proj_with_mqa"),
                 ("self_attn.o_proj",),
                 ("mlp.gate_proj", "mlp.up_proj"),
                 ("mlp.down_proj",),
                 ("mlp.shared_experts.gate_proj", "mlp.shared_experts.up_proj"))


def _align(n: int) -> int:
    return (n + ALIGN - 1) // ALIGN * ALIGN


@dataclass
class BlockPlan:
    """Same fields as adapters/protocol.py:11-20."""
    index: int
    kind: str
    functional: Callable
    kwargs: dict
    host_weights: dict
    adapters: dict
    storage_specs: dict | None = None
    buffer_contract: Any = None
    # this build: a packed pinned image of the block (uint8, plan_layout's
    # nbytes) filled ahead of the session, e.g. by adapter.ArchiveDenseAdapter
    # straight from archive files; Q4SlotSession adopts it instead of packing
    host_image: Any = None


@dataclass
class SlotLayout:
    """Byte layout of one block image; ``entries`` maps a weight name to
    ``('q4', codec, shape, payload_off, payload_bytes, scales_off, scales_bytes)``
    or ``('raw', dtype, shape, off, nbytes)``."""
    nbytes: int
    entries: dict = field(default_factory=dict)


def plan_layout(block: BlockPlan) -> SlotLayout:
    specs = block.storage_specs or {}
    q4 = {name: v for name, v in specs.items() if v["spec"].get("codec") in codecs.FORMATS}
    order, seen = [], set()
    for group in FUSION_GROUPS:
        names = [g + ".weight" for g in group if g + ".weight" in q4]
        if names:
            order.append(names)
            seen.update(names)
    order += [[n] for n in sorted(q4) if n not in seen]
    layout = SlotLayout(0)
    off = 0
    # payload groups, then scale groups: tight inside a group, aligned between
    poffs, soffs = {}, {}
    for names in order:
        off = _align(off)
        for n in names:
            poffs[n] = off
            off += ((q4[n]["spec"]["numel"] + codecs.GROUP - 1) // codecs.GROUP) * codecs.STRIDE
    for names in order:
        off = _align(off)
        for n in names:
            soffs[n] = off
            off += ((q4[n]["spec"]["numel"] + codecs.GROUP - 1) // codecs.GROUP) * 4
    for n in q4:
        spec = q4[n]["spec"]
        groups = (spec["numel"] + codecs.GROUP - 1) // codecs.GROUP
        layout.entries[n] = ("q4", spec["codec"], tuple(spec["shape"]), poffs[n],
                             groups * codecs.STRIDE, soffs[n], groups * 4)
    raw = {k: t for k, t in block.host_weights.items() if not k.startswith("@")}
    for n in sorted(raw):
        off = _align(off)
        t = raw[n]
        layout.entries[n] = ("raw", t.dtype, tuple(t.shape), off, t.numel() * t.element_size())
        off += t.numel() * t.element_size()
    layout.nbytes = _align(off)
    return layout


def _part(block: BlockPlan, name: str, part: str) -> torch.Tensor:
    return block.host_weights[block.storage_specs[name]["parts"][part]]


def pack_image(block: BlockPlan, layout: SlotLayout, out: torch.Tensor) -> None:
    """Write a block's storage into ``out`` (uint8, layout.nbytes) in slot layout."""
    out.zero_()
    for name, e in layout.entries.items():
        if e[0] == "q4":
            _, _, _, po, pb, so, sb = e
            out[po:po + pb].copy_(_part(block, name, "payload"))
            out[so:so + sb].copy_(_part(block, name, "scales").view(torch.uint8))
        else:
            _, dtype, shape, o, nb = e
            out[o:o + nb].copy_(block.host_weights[name].contiguous().view(torch.uint8).reshape(-1))


def views_of(buffer: torch.Tensor, layout: SlotLayout) -> dict:
    """Weight views over a device (or host) image: Q4Weight for 4-bit
    matrices, Q4Experts for packed 3-D expert stacks [E, N, K]."""
    from .moe import Q4Experts
    views = {}
    for name, e in layout.entries.items():
        if e[0] == "q4":
            _, codec, shape, po, pb, so, sb = e
            payload, scales = buffer[po:po + pb], buffer[so:so + sb].view(torch.float32)
            if len(shape) == 3:
                views[name] = Q4Experts(payload, scales, shape[0], shape[1], shape[2], codec)
            else:
                views[name] = Q4Weight(payload, scales, shape, codec)
        else:
            _, dtype, shape, o, nb = e
            views[name] = buffer[o:o + nb].view(dtype).view(shape)
    return views


class _Lease:
    def __init__(self, session, block, token):
        self.session, self.block, self.token = session, block, token

    def __call__(self):
        raise RuntimeError("slot weights require an explicit consumer borrow context")

    def borrow(self, phase):
        return self.session.borrow(self.block, phase, token=self.token)


class Q4SlotSession:
    """Two (or more) device slots of packed layer images with one-layer lookahead."""

    asynchronous = True

    def __init__(self, blocks, device, *, host_budget_bytes, device_budget_bytes, slots=2,
                 prefetch=True, pin=True, image_loader=None):
        self.device = torch.device(device)
        if self.device.type != "cuda":
            raise ValueError("unsupported_capability: the 4-bit slot session requires a GPU device")
        self.blocks = list(blocks)
        if not self.blocks or len({b.index for b in self.blocks}) != len(self.blocks):
            raise ValueError("slot session needs a nonempty unique ordered block plan")
        self.layouts = {id(b): plan_layout(b) for b in self.blocks}
        self.capacity = max(l.nbytes for l in self.layouts.values())
        self.host_bytes = sum(l.nbytes for l in self.layouts.values())
        if self.host_bytes > host_budget_bytes:
            raise MemoryError("resource_budget: pinned block images exceed the host limit")
        if self.capacity * slots > device_budget_bytes:
            raise MemoryError("resource_budget: device slots exceed the device limit")
        if slots < 1 or (len(self.blocks) > 1 and slots < 2):
            raise MemoryError("resource_budget: a multi-block plan needs two slots")
        self.positions = {id(b): i for i, b in enumerate(self.blocks)}
        self.prefetch = prefetch
        # image_loader(block, layout, out) fills a block's image itself (an
        # archive streams its files straight into the pinned buffer);
        # default: pack the block's host tensors
        fill = image_loader or pack_image
        self.images = {}
        for b in self.blocks:
            nbytes = self.layouts[id(b)].nbytes
            img = getattr(b, "host_image", None)
            if img is not None and image_loader is None:
                # a prefilled image of this layout (pinned when the session pins)
                if img.dtype != torch.uint8 or img.numel() != nbytes or img.device.type != "cpu" \
                        or (pin and not img.is_pinned()):
                    raise ValueError("block host_image does not match its slot layout")
            else:
                img = torch.empty(nbytes, dtype=torch.uint8, pin_memory=pin)
                fill(b, self.layouts[id(b)], img)
            self.images[id(b)] = img
        self.pinned_capacity_bytes = self.host_bytes if pin else 0
        self.upload_capacity = 0
        with torch.cuda.device(self.device):
            self.copy_stream = torch.cuda.Stream(device=self.device)
            self.slots = []
            for i in range(slots):
                raw = torch.empty(self.capacity + ALIGN, dtype=torch.uint8, device=self.device)
                buf = raw.narrow(0, (-raw.data_ptr()) % ALIGN, self.capacity)
                self.slots.append({"id": i, "buffer": buf, "block": None, "ready": None,
                                   "consumed": None, "active": False, "last_use": -1, "views": {}})
            self.copy_stream.wait_stream(torch.cuda.current_stream(self.device))
        self._run_lock = threading.Lock()
        self._borrow_lock = threading.Lock()
        self._token = None
        self._owner = None
        self.closed = False
        self.poisoned = False
        self.generation = 0
        self.reloads = self.hits = 0
        self.transferred_bytes = self.actual_h2d_bytes = 0
        self.trace = []
        self.copy_records = []
        self._clock = 0

    # -- run scope ----------------------------------------------------------
    @contextmanager
    def run(self):
        if self.closed or self.poisoned:
            raise RuntimeError("slot session is closed or poisoned")
        if not self._run_lock.acquire(blocking=False):
            raise RuntimeError("concurrent/reentrant session use is unsupported")
        self._owner, self._token = threading.get_ident(), object()
        try:
            yield
        except BaseException:
            self.poisoned = True
            raise
        finally:
            # a failed drain or copy finalisation poisons the session too
            # (prefetch.py:115-131); the run capability is released either way
            try:
                torch.cuda.synchronize(self.device)
                self._finalize_copies()
            except BaseException:
                self.poisoned = True
                raise
            finally:
                self._owner = self._token = None
                self._run_lock.release()

    def reloader(self, block):
        if self._owner != threading.get_ident() or self._token is None:
            raise RuntimeError("reloader creation requires the active session owner")
        if id(block) not in self.positions:
            raise ValueError("block does not belong to this session")
        return _Lease(self, block, self._token)

    # -- slots --------------------------------------------------------------
    def _find(self, block):
        return next((s for s in self.slots if s["block"] is block), None)

    def _victim(self):
        free = [s for s in self.slots if not s["active"]]
        if not free:
            raise RuntimeError("no inactive slot available")
        return min(free, key=lambda s: (s["block"] is not None, s["last_use"], s["id"]))

    def _enqueue(self, block, slot):
        img = self.images[id(block)]
        layout = self.layouts[id(block)]
        self.generation += 1
        record = {"block": block.index, "slot": slot["id"], "generation": self.generation,
                  "overwrote_block": slot["block"].index if slot["block"] is not None else None,
                  "bytes": layout.nbytes}
        slot.update(block=block)
        with torch.cuda.stream(self.copy_stream):
            if slot["consumed"] is not None:
                self.copy_stream.wait_event(slot["consumed"])
            start = torch.cuda.Event(enable_timing=True)
            ready = torch.cuda.Event(enable_timing=True)
            start.record(self.copy_stream)
            slot["buffer"][:layout.nbytes].copy_(img, non_blocking=True)
            ready.record(self.copy_stream)
        slot["ready"] = ready
        slot["views"] = views_of(slot["buffer"], layout)
        record.update(start_event=start, ready_event=ready)
        self.copy_records.append(record)
        self.transferred_bytes += layout.nbytes
        self.actual_h2d_bytes += layout.nbytes

    @contextmanager
    def borrow(self, block, phase, *, token):
        if self.closed or self.poisoned:
            raise RuntimeError("slot session is closed or poisoned")
        if token is not self._token or token is None or not self._run_lock.locked():
            raise RuntimeError("slot borrow requires the active run capability")
        if phase not in ("forward", "backward"):
            raise ValueError("unknown slot consumer phase")
        if not self._borrow_lock.acquire(blocking=False):
            raise RuntimeError("concurrent/reentrant slot borrow is unsupported")
        slot = None
        try:
            slot = self._find(block)
            hit = slot is not None
            if not hit:
                slot = self._victim()
                self._enqueue(block, slot)
            slot["active"] = True
            self._clock += 1
            slot["last_use"] = self._clock
            compute = torch.cuda.current_stream(self.device)
            compute.wait_event(slot["ready"])
            self.reloads += 1
            self.hits += int(hit)
            rec = {"block": block.index, "phase": phase, "slot": slot["id"], "cache_hit": hit,
                   "next_prefetched": None}
            self.trace.append(rec)
            if self.prefetch:
                nxt = self.positions[id(block)] + (1 if phase == "forward" else -1)
                if 0 <= nxt < len(self.blocks):
                    nb = self.blocks[nxt]
                    if self._find(nb) is None and any(not s["active"] for s in self.slots):
                        self._enqueue(nb, self._victim())
                        rec["next_prefetched"] = nb.index
            yield slot["views"]
        except BaseException:
            self.poisoned = True
            raise
        finally:
            try:
                if slot is not None and slot["active"]:
                    # the slot may be overwritten only after this event; if it
                    # cannot be recorded the slot stays active and the session
                    # is poisoned (nf4_cuda_pool.py:543-565)
                    try:
                        consumed = torch.cuda.Event()
                        consumed.record(torch.cuda.current_stream(self.device))
                    except BaseException:
                        self.poisoned = True
                        raise
                    slot["consumed"] = consumed
                    slot["active"] = False
            finally:
                self._borrow_lock.release()

    def invalidate(self):
        """Forget which blocks the slots hold, so the next borrow of every
        block copies its image again (a cold start; used to time the copy of
        a layer that a previous step left in a slot).  Outside ``run()``."""
        if self._run_lock.locked():
            raise RuntimeError("cannot invalidate slots during a run")
        for slot in self.slots:
            slot["block"] = None
            slot["views"] = {}

    def _finalize_copies(self):
        done = []
        for r in self.copy_records:
            row = {k: v for k, v in r.items() if not k.endswith("_event")}
            row["copy_cuda_ms"] = r["start_event"].elapsed_time(r["ready_event"])
            row["h2d_gbps"] = r["bytes"] / max(row["copy_cuda_ms"], 1e-9) / 1e6
            done.append(row)
        self.copy_records.clear()
        self.completed_copies = getattr(self, "completed_copies", []) + done

    def runtime_metadata(self):
        if self._run_lock.locked():
            raise RuntimeError("slot timing requires a completed run")
        return {"mode": "packed_q4_slots_one_layer_prefetch_lru", "slots": len(self.slots),
                "capacity_per_slot_bytes": self.capacity, "cache_hits": self.hits,
                "borrow_count": self.reloads, "copy_trace": getattr(self, "completed_copies", []),
                "lifetime": "ready before use; consumed after complete functional/VJP+gradaccum "
                            "before overwrite"}

    def close(self):
        if self._run_lock.locked() or self._borrow_lock.locked():
            raise RuntimeError("cannot close an active slot session/lease")
        if not self.closed:
            # a failed drain poisons the session and keeps its buffers, so a
            # later close() can retry the cleanup
            try:
                torch.cuda.synchronize(self.device)
            except BaseException:
                self.poisoned = True
                raise
            self.slots.clear()
            self.images.clear()
            self.closed = True


class ResidentSession:
    """All block images resident on the device (no streaming): the reference's
    ``resident=True`` engine mode (engine.py:36-41) for the 4-bit path, and the
    baseline the streamed session is timed against."""

    asynchronous = False

    def __init__(self, blocks, device):
        self.device = torch.device(device)
        self.blocks = list(blocks)
        self.layouts = {id(b): plan_layout(b) for b in self.blocks}
        self.buffers, self.views = {}, {}
        for b in self.blocks:
            lay = self.layouts[id(b)]
            img = torch.empty(lay.nbytes, dtype=torch.uint8)
            pack_image(b, lay, img)
            dev = img.to(self.device)
            self.buffers[id(b)] = dev
            self.views[id(b)] = views_of(dev, lay)
        self.reloads = 0
        self.capacity = max(l.nbytes for l in self.layouts.values())
        self.host_bytes = 0
        self.transferred_bytes = self.actual_h2d_bytes = 0
        self.pinned_capacity_bytes = self.upload_capacity = 0
        self.trace = []

    @contextmanager
    def run(self):
        yield

    def reloader(self, block):
        views = self.views[id(block)]

        def load():
            self.reloads += 1
            return views
        return load

    def close(self):
        self.buffers.clear()
        self.views.clear()


def make_archive_block(reader, index: int, *, heads: int, kv_heads: int, head_dim: int,
                       eps: float, rank: int, alpha: float, targets, device, functional=None,
                       generator=None, prefix: str | None = None, qk_norm: bool = False) -> BlockPlan:
    """A BlockPlan for layer ``index`` of an ``archive.ArchiveReader``: storage
    specs from the archive manifest, raw entries as meta tensors (layout only);
    pass ``reader.image_loader(prefix)`` to the session to fill its image."""
    from .dense import dense_block, lora_kwargs
    from .lora import create_lora_for_block
    prefix = prefix if prefix is not None else f"model.layers.{index}."
    host, specs = reader.block_host_weights(prefix)
    shapes = {n: tuple(v["spec"]["shape"]) for n, v in specs.items()}
    adapters = create_lora_for_block(index, "full_attention", shapes, rank=rank, alpha=alpha,
                                     device=device, targets=tuple(targets), architecture="llama",
                                     generator=generator)
    kwargs = {"heads": heads, "kv_heads": kv_heads, "head_dim": head_dim, "eps": eps,
              **lora_kwargs(adapters)}
    if qk_norm:
        kwargs["qk_norm"] = True
    return BlockPlan(index, "full_attention", functional or dense_block, kwargs, host, adapters,
                     specs)


def make_dense_block(index: int, weights: dict, *, codec: str, heads: int, kv_heads: int,
                     head_dim: int, eps: float, rank: int, alpha: float, targets, device,
                     functional=None, generator=None, qk_norm: bool = False, moe=None,
                     expert_lora_rank: int = 0, expert_lora_alpha: float = 16.0) -> BlockPlan:
    """Encode one dense decoder layer (``weights``: name -> CPU fp32/bf16 tensor,
    HF names without the ``model.layers.{i}.`` prefix) into a BlockPlan whose
    host weights are the flattened 4-bit records (codecs.flatten layout of the
    reference: ``@<name>/payload``, ``@<name>/scales``) plus raw norm vectors.

    A Qwen3-MoE layer (``moe`` = ``{num_experts, top_k, norm_topk_prob}``)
    stores its packed ``mlp.experts.gate_up_proj [E, 2I, H]`` /
    ``mlp.experts.down_proj [E, H, I]`` stacks 4-bit in the same image, so the
    whole decoder layer, every expert included, moves through the slot as in
    qwen3_moe.py:146-152; the router ``mlp.gate.weight`` stays bf16.
    ``expert_lora_rank`` > 0 adds per-expert LoRA on gate|up and down."""
    from .dense import dense_block, lora_kwargs
    from .lora import create_lora_for_block
    host, specs = {}, {}
    for name, t in weights.items():
        if name != "mlp.gate.weight" and t.dim() in (2, 3) and t.numel() >= codecs.GROUP:
            rec = codecs.encode(t.reshape(-1, t.shape[-1]).contiguous(), codec)
            specs[name] = {"spec": dict(rec.spec, shape=list(t.shape)), "parts": {}}
            for part, tensor in rec.parts.items():
                key = f"@{name}/{part}"
                host[key] = tensor
                specs[name]["parts"][part] = key
        else:
            host[name] = t.to(torch.bfloat16).contiguous()
    shapes = {n: tuple(t.shape) for n, t in weights.items() if t.dim() == 2}
    adapters = create_lora_for_block(index, "full_attention", shapes, rank=rank, alpha=alpha,
                                     device=device, targets=tuple(targets), architecture="llama",
                                     generator=generator)
    if moe is not None and expert_lora_rank:
        from .moe import make_expert_lora
        E, I2, H = weights["mlp.experts.gate_up_proj"].shape
        adapters["mlp.experts.gate_up_proj"] = make_expert_lora(
            "mlp.experts.gate_up_proj", E, H, I2, rank=expert_lora_rank, alpha=expert_lora_alpha,
            device=device, segments=2, generator=generator)
        adapters["mlp.experts.down_proj"] = make_expert_lora(
            "mlp.experts.down_proj", E, I2 // 2, H, rank=expert_lora_rank,
            alpha=expert_lora_alpha, device=device, generator=generator)
    kwargs = {"heads": heads, "kv_heads": kv_heads, "head_dim": head_dim, "eps": eps,
              **lora_kwargs(adapters)}
    if qk_norm:  # Qwen3 (dense.py:128-133); q_norm/k_norm vectors travel as raw entries
        kwargs["qk_norm"] = True
    if moe is not None:
        kwargs["moe"] = dict(moe)
    return BlockPlan(index, "full_attention", functional or dense_block, kwargs, host, adapters,
                     specs)


__all__ = ["BlockPlan", "SlotLayout", "plan_layout", "pack_image", "views_of", "Q4SlotSession",
           "ResidentSession", "make_dense_block", "make_archive_block"]
