"""CPU oracle of the FP8 MoE decode layer — TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import
or run anything here, and only as the checker (or, for cpu_baseline, as the
timed CPU restatement). The product path (vibe-megakernel_amd/) never calls it.

Contents:
  formats.py  FP8 E4M3 weight/activation codecs   megabench/tasks/quantization.py:54-131
  routing.py  sigmoid group-limited and softmax    megabench/tasks/frontier.py:229-242,
              top-k routing                        megabench/tasks/distributed.py:174-176,
                                                   megabench/tasks/references/moe.py:68-70
  layer.py    the MoE block with the reference's   megabench/tasks/frontier.py:180-186,335-354
              BF16 rounding schedule, and the
              FP32 ("widened") oracle              megabench/tasks/oracle.py:1-53
  metrics.py  the band rule and the layer checks   megabench/harness/correctness.py:64-85,469-536
  codec.c     plain-C restatement of the byte and  (same citations as formats.py/routing.py,
              integer parts: E4M3/BF16 rounding,    megabench/tasks/megamoe.py:138-149)
              stable top-k selection, histogram
              and stable permutation

How each function is pinned is stated in its docstring; the pins live in
tests/test_oracle_*.py.
"""
