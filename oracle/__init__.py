"""CPU oracle for the TurboQuant packed decode path -- TEST INFRASTRUCTURE ONLY.

This package restates, on the CPU, the reference's algorithm for the three
pieces of the hot path so the HIP implementation in ``winnow_amd`` can be
checked against it:

* ``oracle.packing``    -- LSB-first bit packing (reference ``turboquant_kv/packing.py``)
* ``oracle.quantizer``  -- Lloyd-Max codebook, seeded rotation, quantize
                           (reference ``turboquant_kv/cache.py:62-131``)
* ``oracle.attention``  -- reconstruct / explicit / tiled compressed-domain
                           attention, split merge, paged builders
                           (reference ``turboquant_kv/packed_attention.py:114-377``)
* ``oracle.append``     -- quantize + pack + page scatter of ``PagedPackedCache.update``
                           (reference ``turboquant_kv/packed_backend.py:136-170``)

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline leg
may import this package, and only as the checker (or the timed CPU baseline),
never as the product path.  ``winnow_amd`` never imports it.

Pinning status of each function is recorded in the module docstrings; the
checks that pin them live in ``tests/test_oracle_*.py``.
"""
