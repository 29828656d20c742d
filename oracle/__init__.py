"""CPU oracle for the smooth-attn hot path — TEST INFRASTRUCTURE ONLY.

Nothing in the product (``smooth-attn_amd/``) imports this package.  Only
``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg
use it, and only as the checker (or as the timed CPU baseline), never as the
thing that is measured or shipped.

Modules
-------
``eager``  torch-CPU restatement of the reference's eager formulas (the
           reference's own CPU path, ``implementation="eager"``), in fp32 by
           default and fp64 on request.  Every function cites the reference
           file:line it restates.
``brute``  numpy float64 scalar loops over tiny inputs.  They pin ``eager``
           independently of torch (closed forms evaluated element by element).
``paging`` seeded builders of paged KV caches (sequential and shuffled block
           tables) mirroring the reference tests' cache builders.

Parity status of each function is recorded in its docstring ("pinned by: …").
"""
