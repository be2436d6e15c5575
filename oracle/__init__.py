"""CPU oracle for the baretile hot path — TEST INFRASTRUCTURE ONLY.

Nothing in the product (``baretile_amd``) imports this package. Only ``tests/``,
``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg use it, and only
as the checker (or as the timed CPU baseline), never as the thing measured or shipped.

Modules:
  bfp        bf16 rounding and the block-float (bfp8/bfp4) rules, values and bits
  ops        matmul and attention, as the reference's tests state them
  llama_ref  the NumPy Llama decoder (the reference's NumPy branch of models/llama.py)

Each function cites the reference file:line it restates. Pinning (how each function is
checked against golden vectors, closed forms or an independent library) is listed in
each module's header; a function without such a check says "parity unpinned".
"""
