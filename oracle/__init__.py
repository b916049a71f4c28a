"""CPU oracle for the paged fused-MoE path — TEST INFRASTRUCTURE ONLY.

This package is the checker, never the product. Only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
import it; the library under ``wisp_amd/`` never does, and it fails loudly
when its HIP extension is missing instead of falling back to anything here.

Modules
-------
``pager``   Restatement of the reference pager (``WispMoEState.ensure_resident``
            and the greedy sub-batching of ``_wisp_forward_cuda_paged``) in plain
            CPython, so set iteration order is CPython's own.
``moe``     Routing (softmax -> top-k -> renorm) and the SwiGLU expert MLP with
            the routing-order combine, in float64/float32 on the CPU.

Pinning status of each function is stated in its module header.
"""
