"""CPU oracle for the stick-relayout and decode-attention path.

THIS PACKAGE IS TEST INFRASTRUCTURE.  Only ``tests/``, ``__graft_entry__.smoke()``
and the ``cpu_baseline`` leg of ``bench.py`` may import it, and only as the
checker (or as the timed CPU baseline).  The product package ``torch_spyre_amd``
never imports it and has no CPU fallback.

Modules
-------
layout     SpyreTensorLayout semantics (default tiling, dim_order, explicit
           device_size/stride_map) and the DMA stride-info generation that the
           reference runs for host<->device relayout, plus a numpy executor of
           those loop nests.
relayout   closed forms of the three stick relayouts and the D2D restickify.
attention  the SDPA decode semantics (fp64 restatement of the reference's
           decomposition, torch CPU fp32 SDPA path) and paged-KV gathering.
kv         the ``overwrite`` (narrow + copy) semantics used for KV-cache writes.

Every function cites the reference file:line it restates (paths relative to the
reference repository root).  Parity pins for each function are listed in the
module docstrings; a function with no pin says "parity unpinned".
"""
