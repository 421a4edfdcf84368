"""CPU oracle for the SpillTune per-layer NF4 LoRA training path.

TEST INFRASTRUCTURE ONLY.  Nothing under ``spilltune_amd`` imports this
package: only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline``
leg of ``bench.py`` use it, and only as the checker (or, for the CPU baseline,
as the timed restatement of the reference's CPU training path).

* ``oracle.codec``  -- C restatement of the 4-bit storage decode/encode
  (``oracle/codec.c``), loaded with ctypes from ``oracle/_build``.
* ``oracle.layer``  -- PyTorch-CPU restatement of the LoRA projection, the
  dense (Llama) decoder block, the streaming recompute driver, the chunked
  causal-LM terminal and the AdamW update.

Pinning status (what each function is checked against) is listed in the
module headers; every function has an independent pin.
"""
