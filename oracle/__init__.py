"""CPU oracle for the Gemma-4 MoE decode path — TEST INFRASTRUCTURE ONLY.

This package restates, on the CPU, what the JAX reference
(YLiu95/kaggle-tpu-inference, gemma4_tpu/model.py) computes, so the HIP path
can be checked against it.  It is imported only by tests/, by
__graft_entry__.smoke() and by bench.py's cpu_baseline leg; the product
(kaggle-tpu-inference_amd/gemma4_mi) never imports or calls it.

Modules:
  philox.py  numpy restatement of the weight generator (Philox4x32-10 +
             Box-Muller) and the per-tensor key derivation.
  twin.py    torch-CPU restatement of model.py: primitives, attention, router,
             MoE (decode "slice" path and dense prefill path), layer, forward,
             masks, greedy sampling, cache.

Rounding recipe (the reference leaves accumulation order and fusion to XLA, so
these points define it; the GPU path follows the same recipe):
  * every einsum: exact-ish f64 accumulation, result rounded f64 -> f32 -> bf16;
  * every elementwise jnp op on bf16 operands: computed in f32, rounded to bf16;
    gelu and rms_norm count as one op each;
  * rms_norm: sum of squares exact (f64), mean = f32(sum)/H in f32,
    scale = f32(1/sqrt(f64(mean + eps))), out = bf16(x * scale * w) in f32;
  * softmax in f32 with max subtraction; the router's exp is evaluated in f64
    and rounded to f32 and its sums are exact, so top-k indices are
    reproducible bit for bit;
  * RoPE cos/sin: f32(cos_f64(f32(pos) * inv_freq_f32)), then bf16.

Parity status per function is listed in the module docstrings; every function
here is checked by at least one test in tests/ (closed form, known answer,
HF transformers sub-module, brute force or invariant).
"""
