"""TEST INFRASTRUCTURE ONLY -- the CPU oracle for the causal pre-norm block path.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import
this package, and only as the checker (or, for cpu_baseline, the timed CPU
reference); the product path in gpu-kernel-for-transformer_amd/ never imports
it and has no CPU fallback.

Contents
  baseline.py   restated BaselineTransformer (torch, FP32, CPU), input
                generation and weight copy (torch_transformer_benchmark.py:204-317,
                :1151-1220)
  accuracy.py   the reference's elementwise OR accuracy rule
                (torch_transformer_benchmark.py:1223-1304)
  numpy_ref.py  float64 NumPy brute force of the same forward, written from
                the formulas (explicit loops for attention), used to pin
                baseline.py on tiny inputs

Pinning (what checks each function, see tests/test_oracle.py)
  BaselineTransformer   numpy_ref float64 brute force on tiny inputs;
                        causal-prefix invariance; batch independence;
                        S=1 closed form out_proj(v_proj(LN(x))); LN row
                        statistics; a planted-mistake test (wrong causal
                        diagonal, tanh GELU, missing scale) that the brute
                        force must reject
  compare_outputs       closed-form unit cases (boundary |d| == atol passes,
                        NaN/inf fail, ref == 0 falls back to atol, the OR is
                        not isclose's sum)
  generate_random_case  shape/dtype/seed determinism and the padding
                        contract (lengths in [round(S*(1-r)), S])
  numpy_ref             textbook identities (softmax rows sum to 1, erf GELU
                        against math.erf, LayerNorm against the definition)
"""
