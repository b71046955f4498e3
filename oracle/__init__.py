"""CPU oracle of the batch-1 ternary decode path.

TEST INFRASTRUCTURE ONLY. Nothing in the product (trixium_amd/) imports, calls or links this
package; only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use it, as the
checker the HIP path is compared against (and as the timed CPU baseline).

Contents (each function cites the reference file:line it restates):
  bitexact.py   integer engine contract: fp16 split, B/R choice, exact ternary/Q8 matvec,
                group sums, the power-of-two int8 activation quantizer
  floatref.py   float reference of the decoder (fastref numerics with FloatModel's step and
                state semantics): dense Qwen3 and the hybrid Gated-DeltaNet/attention model;
                ShapeSample, the same step on random weights of a large shape (CPU timing)
"""
