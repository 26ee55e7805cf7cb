"""CPU oracle for the selas_amd hot path: TEST INFRASTRUCTURE ONLY.

A restatement of the reference algorithms (tcox-coding/selas), used by
``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` as the checker. The product package ``selas_amd`` never imports
anything from here.

Modules:
  nf4       NF4 encode/decode in numpy (and the C restatement nf4_ref.c via ctypes),
            plus the fp32 -> bf16/fp16 roundings they use.
  segments  the elementwise segments and their primitives, torch on the CPU.
  flux      the block composition (double/single/final) and the step, torch on the CPU.

Parity status of each function (how it is pinned) is listed in each module's
header. Nothing here is "parity unpinned" except where a module says so.
"""
