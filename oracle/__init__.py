"""CPU oracle for the NF4-LoRA projection path. TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import this
package, and only as the checker (or the timed CPU baseline); the product path under
causal-tuner_amd/ never imports it.

Contents (each function cites the reference file:line it restates):
  nf4.py          numpy restatement of the NF4 decode closed form (bit-exact) and of the
                  bitsandbytes quantizer the reference delegates to (parity with
                  bitsandbytes' bits unpinned: the library is absent and the reference's
                  tests store no quantized bytes).
  lora.py         the reference's torch-op sequence for one projection (CPU, bf16) and a
                  float64-accumulated oracle with the reference's bf16 rounding points for
                  xa and low and one final rounding of out and dx.
  mlp.py          the tiled LoRA MLP (SiLU-multiply with its bf16 rounding points, gate/up/
                  down projections, analytic backward) in float64.
  rope.py         the partial GPT-J rotary embedding with its per-product rounding
                  (numpy float32 + explicit round-to-nearest-even).
  rmsnorm.py      row-wise RMS normalization forward/backward (float64 with the
                  reference's rounding points to the activation dtype).
  nf4_dequant.c   plain-C decode, the timed CPU baseline (built by oracle/Makefile).
"""
