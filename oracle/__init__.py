"""CPU oracle for the CARE-KV quantized decode-attention path.

TEST INFRASTRUCTURE ONLY.  This package is a numpy restatement of the
reference algorithm (soeunida/CARE-KV-..., Python/PyTorch prototype) used as
the parity checker for the HIP kernels.  Only ``tests/``,
``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may import
it, and only to check or time; the product package never calls it.

Modules and what pins each one (reference paths are relative to the
reference root):

* ``quant``     -- ``quantizer.py:31-383`` quantize/dequantize/bit packing,
                   ``cache.py:592-718`` int8 scale codes,
                   ``residual_store.py:121-176`` 4/8-bit residual slots.
                   Pinned by closed form (bit positions, round-trip), the
                   reference-held activation arrays (fp32 path, tie
                   exemption) and committed goldens (fp16 path).
* ``cache``     -- ``cache.py:416-904`` paged cache (packed base, int8
                   scales, slot arenas, page metadata).  Pinned by goldens.
* ``store``     -- ``residual_store.py:239-464`` store-time candidate
                   enumeration and selection.  Pinned by goldens.
* ``attention`` -- ``attention.py:96-184,386-957,979-1039`` base attention,
                   exact renormalisation, query-aware K score and the
                   batched joint correction (comb+ex selector).  Pinned by
                   goldens, an fp64 brute force of the exact
                   renormalisation, and the READ=0 / kind=v invariants.
"""
