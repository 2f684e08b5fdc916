"""CPU oracle for the multi-future-drafting hot path (TEST INFRASTRUCTURE ONLY).

This package restates, on the CPU, the algorithms of the reference's hot path so that the HIP
kernels can be checked against them:

  gdn.py          tree gated-delta-rule verification (chunk form and node-by-node recurrence)
  attention.py    K-mode drafter attention (flat and paged KV cache), masked softmax in fp64
  builder.py      ctypes front of csrc/oracle.c: the logits step (top-k with an explicit tie rule and
                  the deterministic log Z), the exact mixture-tree and single-mode best-first heaps,
                  the visibility matrix; loaders of the reference's own C++ builders (oracle/_ref)
  build_oracle.py builds csrc/oracle.c, and oracle/_ref from the reference's sources where present
  synth.py        the seeded synthetic inputs of the benchmark configurations

Only tests, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may import this
package, and only as the checker or the timed CPU baseline. The product library never calls it.
"""
