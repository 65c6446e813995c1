"""Host-side Python mirror of the aot-llm hot-path interface over libaotk.so.

The names follow the reference's runtime (crates/aot-kernels): `matvec`,
`matmul`, `quantize_q8_k`, `dequant_row`, a `Model` holding weights resident
in HBM and a `State` with the KV cache, `forward` / `forward_batch`
(app.rs:32-62 ForwardFn / ForwardBatchFn) and greedy generation
(app.rs:553-610). Everything runs through the HIP library; there is no CPU
fallback: a missing library raises AotkError.
"""
from . import abi, configs  # noqa: F401
from .abi import AotkError  # noqa: F401
from .runtime import (  # noqa: F401
    DeviceBuffer, Model, Sampler, copy_dev, State, Weight, argmax, attention, dequant_rows, gelu_mul, init, matmul, matmul2, matmul_noalloc, matvec, matvec2, matvec3,
    matvec_f32, quantize_q8_0, quantize_q8_k, quantize_rows, rmsnorm, rmsnorm_heads, rope, silu_mul, softmax,
    stream, sync, time_hbm, time_matvec, time_matmul,
)
