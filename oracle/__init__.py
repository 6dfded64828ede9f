"""CPU oracle for the video-DiT attention hot path — TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s
``cpu_baseline`` leg may import this package, and only as the checker (or the
timed CPU baseline), never as the measured or shipped path.  The product
(``avgen_amd``) never imports it.

Modules:

* :mod:`oracle.reference` — numpy restatement of the reference path: 3D
  RoPE (src/avgen/models/rope.py), SDPA with key-padding mask and LSE
  (src/avgen/models/attention.py -> torch SDPA), the flash backward, the
  ring merge and the ring forward/backward loops
  (torch/distributed/tensor/experimental/_context_parallel/_attention.py),
  contiguous sharding (src/avgen/parallel/context.py), the query-dependent
  masks (temporal neighbourhoods, src/avgen/models/blocks.py:54-104; packed
  sequences, src/avgen/data/packing.py:136-200) and the FLOP
  convention (src/avgen/simulate/compute.py).  Attention math is float64;
  the RoPE rotation mirrors the reference's float32 elementwise chain bit for
  bit and rounds to bf16.
* :mod:`oracle.torch_path` — the same reference path written in PyTorch CPU
  ops (the reference *is* PyTorch code); used as the timed CPU baseline and
  as an independent cross-check of :mod:`oracle.reference`.

Pinning (what makes these functions trustworthy, tested in
``tests/test_oracle.py``): closed forms and textbook special cases, agreement
of the two independent implementations (numpy float64 vs PyTorch's own CPU
SDPA kernel and autograd), finite differences, and invariants (chunked+merged
== unchunked, merge associativity, RoPE norm preservation / relative-position
property / identity at zero coordinates, exact zeros for masked keys).  The
reference ships no golden vectors for this path, so none can be replayed;
see the oracle tests for which check pins which function.  No function here
is "parity unpinned".
"""
