"""TEST INFRASTRUCTURE ONLY: CPU oracle of the Parrot inference MoE path.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s
``cpu_baseline`` leg may import this package, and only as the checker (or,
for the CPU baseline, as the timed reference-equivalent path).  The product
(``parrot`` package, C ABI) never imports it.

  routing      -- C closed form of top-2 / stable slots / capacity / overflow
                  (oracle/route_group.c) plus pure-Python brute force
  layers       -- fp32 RMSNorm, Block AttnRes depth mix, SwiGLU, MoE layer
  parrot_fp32  -- functional fp32 forward / prefill / decode of the full model
"""
