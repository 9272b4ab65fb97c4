"""CPU oracle for the RidgeFill fill path (TEST INFRASTRUCTURE, not product code).

A PyTorch-on-CPU restatement of the reference algorithm for the hot path, written for checking the
HIP kernels. Only `tests/`, `__graft_entry__.smoke()` and `bench.py`'s `cpu_baseline` leg may import
it, and only as the checker or as the reported CPU baseline -- never as the thing measured or shipped.
The product (`rfill`) never imports this package.

Modules and the reference code they restate (paths relative to the reference repository):
  ops.py    norms, RoPE, attention, causal conv, chunked / recurrent gated delta rule
            (code/kva/ops.py:14-277)
  model.py  layer-wise forward of Llama-3.1 / Qwen3 / Qwen3.5 over explicit caches: fill, fill_kv,
            layer, layer_rows (code/kva/model.py:105-572)
  kva.py    Arm, Projector (+ its safetensors format), run_lower, finish's fill loop, rounded_tail
            (code/kva/kva.py:79-193, 261-300, 319-460)
  ridge.py  RidgeStats, RidgeFit, residual, combine and fit_sweep's capture sums
            (code/kva/ridge.py:19-156, code/scripts/fit_sweep.py:62-166)

How each function is pinned (tests/test_oracle_*.py):
  * model math against transformers' own LlamaForCausalLM / Qwen3ForCausalLM / Qwen3_5ForCausalLM
    tiny random models (logits, and every layer's K/V cache, conv state and recurrent state), the
    oracle the reference's own tests use;
  * chunked delta rule against the token-by-token recurrence (a closed form), causal conv against
    F.conv1d + SiLU;
  * ridge fit against an independent augmented least-squares solve, OLS as lambda -> 0, exact recovery
    of a noiseless linear map, and the sums against a naive recomputation;
  * finish() against the invariants the reference tests hold (tail = N is the exact forward bitwise;
    oracle fill = exact prefill; every prefix row exact = exact cache);
  * composed finish() outputs, RidgeFit.layer and the capture shift convention against golden vectors
    written by tests/golden/make_golden.py from the reference itself (see that script's header).
"""
