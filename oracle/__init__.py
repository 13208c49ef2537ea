"""CPU oracle for the hot path -- TEST INFRASTRUCTURE ONLY.

This package restates, in torch-CPU fp32/fp64, the arithmetic of each reference kernel that the
HIP library replaces (each function cites the reference file:line it follows).  It is the checker
the parity tests, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg compare the
HIP kernels against; nothing in the product (``pytorchsim-triton-backend_amd/``) imports it, and
the product has no CPU fallback.

How each function is pinned (tests/test_oracle.py):
  rmsnorm, qk_norm_rope     torch.nn.functional.rms_norm / fp64 closed form, constant-row special
                            case, cos=1/sin=0 reduces to the norm, brute-force loops on tiny inputs,
                            golden fixtures of an independent fp64 computation
  softmax_rows              torch.softmax in fp64, rows sum to 1, shift invariance, NaN propagation
  silu_mul                  torch.nn.functional.silu in fp64
  transpose_heads           torch.permute (exact) and a brute-force index loop
  reduce_sum / reduce_max   math.fsum / Python max over the same values
  gemm (+residual)          fp64 matmul, brute-force triple loop on tiny shapes
  quant_rows / quant_weight torch's float8_e4m3fn cast, exhaustive round trip of all 256 codes,
  / gemm_fp8                saturation at 448, brute force on tiny shapes
  flash_attention           fp64 softmax(QK^T * s + causal) V with GQA repeat, V=const -> O=const,
                            row 0 attends only to key 0
  qwen3_layer               composition of the above in the manifest's launch order, checked
                            against an independent fp64 restatement of the Qwen3 block
  moe.*                     (the Qwen3-30B-A3B MoE kernels) torch.sort / torch.topk / torch.cumsum
                            / one-hot sums on the same inputs, brute-force Python loops on tiny
                            inputs, routing invariants (every slot lands in exactly one expert
                            row, dispatch -> grouped GEMM -> combine equals the dense mixture)

Parity for the reference's *execution* arithmetic (its MXU accumulation order and EUP exp inside
the un-vendored Coprocessor model) is unpinned beyond the tolerances its own baselines record;
fp8 has no reference-side pin at all (fp8 is refused on tpuv6e, tests/baselines/tpuv6e.txt:174).
"""
from .kernels import *  # noqa: F401,F403
from .moe import *  # noqa: F401,F403
