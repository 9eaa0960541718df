"""hsdpa: the MI355X (gfx950) attention step of herbert-jit-bf16 behind a C ABI.

The compute path is libhsdpa.so (hand-written HIP kernels, include/hsdpa.h).
This package holds its ctypes binding (binding.py), which mirrors the
reference's AttentionSpec / AttentionCall records, the KV snapshot format and
multi-layer device cache (snapshot.py), and the seeded synthetic workloads
(workloads.py) used by the tests and the benchmark.
"""
from . import workloads  # noqa: F401
from .binding import (  # noqa: F401
    HsdpaError, Plan, Spec, Call, STATUS, library, library_path, attention_torch,
    KvSpec, KvCall, kv_spec, kv_append_raw, kv_append_torch,
    NormRopeSpec, NormRopeCall, GateSpec, GateCall, head_norm_rope_torch, output_gate_torch,
    kv_restore_raw, kv_take_raw, LayerCall, attention_layer_torch,
)
from . import snapshot  # noqa: F401
