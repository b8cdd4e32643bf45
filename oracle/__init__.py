"""CPU oracle for the fused LTX-2.3 DiT block ops.

TEST INFRASTRUCTURE ONLY. This package restates, in numpy, the torch
expressions that plugyawn/opengenie runs when its fused kernels are not used
(the `_torch_*` fallbacks and the torch expressions in the wrappers of
`ltx_serve/triton_ltx_ops.py`). It exists to check the HIP library. Only
`tests/`, `__graft_entry__.smoke()` and the CPU-baseline leg of `bench.py` may
import it; the product package `opengenie_amd` never does.

Every value that torch would hold as bfloat16 is held here as a float32 array
whose values are exactly representable in bfloat16; `numerics.bf16_round` is
applied at exactly the points where torch's result dtype is bfloat16.

`oracle.torch_ref` holds the same expressions written in torch, so that torch
itself evaluates them (on the CPU for the pins, on the GPU for the device
semantics, and on the host cores as bench.py's CPU baseline).

Parity pins (what checks each function; the tests named live in `tests/`):
- numerics.bf16_round: torch CPU float32->bfloat16 conversion, exhaustive
  over structured and random float32 bit patterns (test_oracle_pins.py).
- numerics.e4m3_encode/e4m3_decode: torch CPU float->float8_e4m3fn
  conversion, exhaustive over all 65536 bfloat16 patterns and float32
  boundary sets (test_oracle_pins.py).
- ltx_ops.*: each op against the reference's own torch expression executed
  by torch on the CPU for the shapes of the reference's tests, plus the
  committed golden fixtures in tests/golden (same expressions, stored).
- ltx_ops.rms_norm: torch.nn.functional.rms_norm on the CPU (bounded
  mismatch rate: torch's float32 reduction order is implementation-defined),
  plus closed forms (constant rows).
- ltx_ops.fp8_scaled_mm: torch._scaled_mm on the CPU, and brute-force
  float64 dot products on tiny shapes.
- ltx_ops.video_qk_rmsnorm_rope: the reference test's restatement of split
  RoPE (tests/test_triton_ltx_ops.py:232-249) executed by torch, plus the
  invariants cos=1/sin=0 -> rms_norm*w and sin=1/cos=0 -> a quarter turn.
- ltx_ops.attention: torch.nn.functional.scaled_dot_product_attention in
  float64 on the CPU.
- ltx_ops.gelu_tanh: torch's gelu(approximate='tanh') on the GPU over all
  65536 bfloat16 inputs, bit for bit (test_gpu_parity.py), and on the CPU
  except four inputs where torch's vectorised CPU tanh saturates early.
- ltx_ops.fp8_per_head_quantize: torch's expression (:976-980) on the CPU
  (device="cpu", division by 448) and on the GPU (device="cuda",
  multiplication by float32(1/448), torch's GPU rule for a Python-scalar
  divisor), including NaN heads.
"""
