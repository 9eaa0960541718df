"""ctypes binding of libhsdpa.so (include/hsdpa.h).

The structures mirror the reference's per-layer geometry and per-call records
(src/jit/execution/abi.rs:136-180); the status codes mirror its named
refusals (Decline, src/jit/ir.rs:177-230). Device memory and streams come
from PyTorch, as plumbing only: the arithmetic is the HIP kernels'. There is
no fallback: if libhsdpa.so is missing or fails to load, every call raises.
"""
from __future__ import annotations

import ctypes
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_NAME = "libhsdpa.so"
_lib = None

STATUS = {
    0: "HSDPA_OK", 1: "HSDPA_ERR_EMPTY", 2: "HSDPA_ERR_HEAD_DIM", 3: "HSDPA_ERR_GQA",
    4: "HSDPA_ERR_STRIDE", 5: "HSDPA_ERR_SINK_UNSUPPORTED", 6: "HSDPA_ERR_CAPACITY",
    7: "HSDPA_ERR_WORKSPACE", 8: "HSDPA_ERR_ALIGNMENT", 9: "HSDPA_ERR_NULL", 10: "HSDPA_ERR_HIP",
    11: "HSDPA_ERR_NO_DEVICE", 12: "HSDPA_ERR_BATCH", 13: "HSDPA_ERR_LAYOUT", 14: "HSDPA_ERR_FORM",
    15: "HSDPA_ERR_STATIC_SCRATCH", 16: "HSDPA_ERR_FRAME",
}
STATIC_SCRATCH_BYTES = 32 << 20
FORMS = {"chained": 0, "fused": 1}
KERNELS = {0: "none", 1: "decode", 2: "few_rows", 3: "causal", 4: "causal_split", 5: "decode_rows",
           6: "causal_short", 7: "causal_paired"}
EXPORTS = ["hsdpa_plan_create", "hsdpa_plan_destroy", "hsdpa_workspace_bytes", "hsdpa_attention",
           "hsdpa_status_string", "hsdpa_version", "hsdpa_kv_check", "hsdpa_kv_append",
           "hsdpa_head_norm_rope", "hsdpa_output_gate", "hsdpa_kv_restore", "hsdpa_kv_take",
           "hsdpa_attention_layer", "hsdpa_attention_route", "hsdpa_attention_static",
           "hsdpa_attention_frame"]


class HsdpaError(RuntimeError):
    def __init__(self, code: int, what: str):
        self.code = code
        self.name = STATUS.get(code, f"status {code}")
        super().__init__(f"{what}: {self.name} ({library().hsdpa_status_string(code).decode()})")


class Spec(ctypes.Structure):
    _fields_ = [("heads", ctypes.c_uint64), ("gqa", ctypes.c_uint64), ("head_dim", ctypes.c_uint64),
                ("q_row", ctypes.c_uint64), ("q_head", ctypes.c_uint64), ("out_row", ctypes.c_uint64),
                ("kv_capacity", ctypes.c_uint64), ("kv_stride", ctypes.c_uint64),
                ("grouped", ctypes.c_uint32), ("sink", ctypes.c_uint32), ("form", ctypes.c_uint32),
                ("reserved", ctypes.c_uint32), ("max_rows", ctypes.c_uint64)]


class Call(ctypes.Structure):
    _fields_ = [("q", ctypes.c_void_p), ("keys", ctypes.c_void_p), ("values", ctypes.c_void_p),
                ("output", ctypes.c_void_p), ("rows", ctypes.c_uint64), ("past", ctypes.c_uint64),
                ("scale", ctypes.c_float), ("sink", ctypes.c_float), ("workspace", ctypes.c_void_p),
                ("workspace_bytes", ctypes.c_uint64)]


class FrameCall(ctypes.Structure):
    """hsdpa_frame_call: rows and past as device pointers (AttentionCall, abi.rs:156-180)."""
    _fields_ = [("q", ctypes.c_void_p), ("keys", ctypes.c_void_p), ("values", ctypes.c_void_p),
                ("output", ctypes.c_void_p), ("rows", ctypes.c_void_p), ("past", ctypes.c_void_p),
                ("scale", ctypes.c_float), ("sink", ctypes.c_float), ("workspace", ctypes.c_void_p),
                ("workspace_bytes", ctypes.c_uint64), ("status", ctypes.c_void_p)]


class Route(ctypes.Structure):
    """hsdpa_route: the kernels a call would run."""
    _fields_ = [("main", ctypes.c_uint32), ("main_form", ctypes.c_uint32), ("tail", ctypes.c_uint32),
                ("tail_form", ctypes.c_uint32), ("main_rows", ctypes.c_uint64), ("tail_rows", ctypes.c_uint64),
                ("splits", ctypes.c_uint32), ("launches", ctypes.c_uint32)]


class KvSpec(ctypes.Structure):
    """KvSpec (src/jit/execution/abi.rs:57-73)."""
    _fields_ = [("heads", ctypes.c_uint64), ("head_dim", ctypes.c_uint64), ("stride", ctypes.c_uint64),
                ("capacity", ctypes.c_uint64), ("max_batch", ctypes.c_uint64), ("r16", ctypes.c_uint32),
                ("reserved", ctypes.c_uint32)]


class KvCall(ctypes.Structure):
    """KvCall (src/jit/execution/abi.rs:105-130), rows and past by value."""
    _fields_ = [("keys", ctypes.c_void_p), ("values", ctypes.c_void_p), ("input_keys", ctypes.c_void_p),
                ("input_values", ctypes.c_void_p), ("rows", ctypes.c_uint64), ("past", ctypes.c_uint64)]


class NormRopeSpec(ctypes.Structure):
    _fields_ = [("heads", ctypes.c_uint64), ("head_dim", ctypes.c_uint64), ("head_stride", ctypes.c_uint64),
                ("row_stride", ctypes.c_uint64), ("rotary_dims", ctypes.c_uint64), ("table_row", ctypes.c_uint64),
                ("positions", ctypes.c_uint64), ("plus_one", ctypes.c_uint32), ("reserved", ctypes.c_uint32)]


class NormRopeCall(ctypes.Structure):
    _fields_ = [("data", ctypes.c_void_p), ("weight", ctypes.c_void_p), ("cos", ctypes.c_void_p),
                ("sin", ctypes.c_void_p), ("rows", ctypes.c_uint64), ("past", ctypes.c_uint64),
                ("eps", ctypes.c_float), ("reserved", ctypes.c_float)]


class GateSpec(ctypes.Structure):
    _fields_ = [("width", ctypes.c_uint64), ("attn_row", ctypes.c_uint64), ("gate_row", ctypes.c_uint64)]


class GateCall(ctypes.Structure):
    _fields_ = [("attn", ctypes.c_void_p), ("gate", ctypes.c_void_p), ("rows", ctypes.c_uint64)]


class LayerCall(ctypes.Structure):
    """hsdpa_layer_call: the attention chain of one layer."""
    _fields_ = [(n, ctypes.c_void_p) for n in ("q", "k", "v", "keys", "values", "output", "gate", "q_norm",
                                                "k_norm", "cos", "sin")] + \
               [(n, ctypes.c_uint64) for n in ("rows", "past", "kv_row", "gate_row", "rotary_dims", "table_row",
                                                "positions")] + \
               [("scale", ctypes.c_float), ("eps", ctypes.c_float), ("plus_one", ctypes.c_uint32),
                ("reserved", ctypes.c_uint32), ("workspace", ctypes.c_void_p), ("workspace_bytes", ctypes.c_uint64)]


def library_path() -> str:
    return os.path.join(_HERE, _LIB_NAME)


def library():
    """Load libhsdpa.so (raises OSError when it is not built)."""
    global _lib
    if _lib is None:
        path = library_path()
        if not os.path.exists(path):
            raise OSError(f"{path} is not built: run herbert-jit-bf16_amd/build.py")
        L = ctypes.CDLL(path)
        L.hsdpa_plan_create.argtypes = [ctypes.POINTER(Spec), ctypes.POINTER(ctypes.c_void_p)]
        L.hsdpa_plan_create.restype = ctypes.c_int
        L.hsdpa_plan_destroy.argtypes = [ctypes.c_void_p]
        L.hsdpa_plan_destroy.restype = None
        L.hsdpa_workspace_bytes.argtypes = [ctypes.c_void_p]
        L.hsdpa_workspace_bytes.restype = ctypes.c_uint64
        L.hsdpa_attention.argtypes = [ctypes.c_void_p, ctypes.POINTER(Call), ctypes.c_void_p]
        L.hsdpa_attention.restype = ctypes.c_int
        L.hsdpa_status_string.argtypes = [ctypes.c_int]
        L.hsdpa_status_string.restype = ctypes.c_char_p
        L.hsdpa_version.restype = ctypes.c_uint32
        L.hsdpa_kv_check.argtypes = [ctypes.POINTER(KvSpec)]
        L.hsdpa_kv_check.restype = ctypes.c_int
        L.hsdpa_kv_append.argtypes = [ctypes.POINTER(KvSpec), ctypes.POINTER(KvCall), ctypes.c_void_p]
        L.hsdpa_kv_append.restype = ctypes.c_int
        L.hsdpa_head_norm_rope.argtypes = [ctypes.POINTER(NormRopeSpec), ctypes.POINTER(NormRopeCall),
                                           ctypes.c_void_p]
        L.hsdpa_head_norm_rope.restype = ctypes.c_int
        L.hsdpa_output_gate.argtypes = [ctypes.POINTER(GateSpec), ctypes.POINTER(GateCall), ctypes.c_void_p]
        L.hsdpa_output_gate.restype = ctypes.c_int
        u16p = ctypes.c_void_p
        L.hsdpa_kv_restore.argtypes = [ctypes.POINTER(KvSpec), u16p, ctypes.c_uint64, u16p, u16p, ctypes.c_uint64,
                                       ctypes.c_void_p]
        L.hsdpa_kv_restore.restype = ctypes.c_int
        L.hsdpa_kv_take.argtypes = [ctypes.POINTER(KvSpec), u16p, u16p, u16p, ctypes.c_uint64, ctypes.c_uint64,
                                    ctypes.c_void_p]
        L.hsdpa_kv_take.restype = ctypes.c_int
        L.hsdpa_attention_layer.argtypes = [ctypes.c_void_p, ctypes.POINTER(LayerCall), ctypes.c_void_p]
        L.hsdpa_attention_layer.restype = ctypes.c_int
        L.hsdpa_attention_route.argtypes = [ctypes.c_void_p, ctypes.c_uint64, ctypes.c_uint64, ctypes.POINTER(Route)]
        L.hsdpa_attention_route.restype = ctypes.c_int
        L.hsdpa_attention_static.argtypes = [ctypes.c_void_p, ctypes.POINTER(Call), ctypes.c_void_p]
        L.hsdpa_attention_static.restype = ctypes.c_int
        L.hsdpa_attention_frame.argtypes = [ctypes.c_void_p, ctypes.POINTER(FrameCall), ctypes.c_void_p]
        L.hsdpa_attention_frame.restype = ctypes.c_int
        _lib = L
    return _lib


class Plan:
    """A validated per-layer geometry (hsdpa_plan_create). Mirrors the
    reference's mount: AttentionSpec plus the cache reserve."""

    def __init__(self, heads: int, gqa: int, head_dim: int, kv_capacity: int, q_row: int | None = None,
                 q_head: int | None = None, out_row: int | None = None, kv_stride: int | None = None,
                 grouped: bool = False, sink: bool = False, form: str | int = "chained", max_rows: int = 0):
        form_code = FORMS[form] if isinstance(form, str) else int(form)
        self.spec = Spec(heads, gqa, head_dim,
                         heads * head_dim if q_row is None else q_row,
                         head_dim if q_head is None else q_head,
                         heads * head_dim if out_row is None else out_row,
                         kv_capacity, kv_capacity * head_dim if kv_stride is None else kv_stride,
                         int(grouped), int(sink), form_code, 0, max_rows)
        self._h = ctypes.c_void_p()
        rc = library().hsdpa_plan_create(ctypes.byref(self.spec), ctypes.byref(self._h))
        if rc != 0:
            raise HsdpaError(rc, "hsdpa_plan_create")

    @property
    def handle(self):
        return self._h

    @property
    def workspace_bytes(self) -> int:
        return int(library().hsdpa_workspace_bytes(self._h))

    def route(self, rows: int, past: int) -> dict:
        """The kernels a call of `rows` rows after `past` positions would run."""
        r = Route()
        rc = library().hsdpa_attention_route(self._h, rows, past, ctypes.byref(r))
        if rc != 0:
            raise HsdpaError(rc, "hsdpa_attention_route")
        return {"main": KERNELS[r.main], "main_form": "fused" if r.main_form else "chained",
                "tail": KERNELS[r.tail], "tail_form": "fused" if r.tail_form else "chained",
                "main_rows": r.main_rows, "tail_rows": r.tail_rows, "splits": r.splits, "launches": r.launches}

    def attention_raw(self, q: int, keys: int, values: int, output: int, rows: int, past: int, scale: float,
                      workspace: int, workspace_bytes: int, stream: int = 0, sink: float = 0.0) -> None:
        call = Call(q, keys, values, output, rows, past, scale, sink, workspace, workspace_bytes)
        rc = library().hsdpa_attention(self._h, ctypes.byref(call), ctypes.c_void_p(stream))
        if rc != 0:
            raise HsdpaError(rc, "hsdpa_attention")

    def attention_frame_raw(self, q: int, keys: int, values: int, output: int, rows_ptr: int, past_ptr: int,
                            scale: float, workspace: int, workspace_bytes: int, status_ptr: int = 0,
                            stream: int = 0, sink: float = 0.0) -> None:
        """hsdpa_attention_frame: rows and past are device pointers the kernels read."""
        call = FrameCall(q, keys, values, output, rows_ptr, past_ptr, scale, sink, workspace, workspace_bytes,
                         status_ptr)
        rc = library().hsdpa_attention_frame(self._h, ctypes.byref(call), ctypes.c_void_p(stream))
        if rc != 0:
            raise HsdpaError(rc, "hsdpa_attention_frame")

    def close(self) -> None:
        if self._h:
            library().hsdpa_plan_destroy(self._h)
            self._h = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def attention_torch(plan: Plan, q, k, v, out, rows: int, past: int, scale: float, workspace, stream=None,
                    sink: float = 0.0) -> None:
    """Enqueue the node on torch device tensors (uint16/int16/bfloat16 views of
    bf16 data). `workspace` is a uint8 device tensor of plan.workspace_bytes;
    `sink` is the sink's score, read when the plan has the sink flag."""
    import torch

    for t in (q, k, v, out, workspace):
        if not t.is_cuda or not t.is_contiguous():
            raise ValueError("tensors must be contiguous device tensors")
    s = torch.cuda.current_stream() if stream is None else stream
    plan.attention_raw(q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), rows, past, scale,
                       workspace.data_ptr(), workspace.numel() * workspace.element_size(), s.cuda_stream, sink)


def kv_spec(heads: int, head_dim: int, capacity: int, max_batch: int, stride: int | None = None,
            r16: bool = False) -> KvSpec:
    """A KV reserve geometry, validated like KvSpec::validate (raises HsdpaError)."""
    spec = KvSpec(heads, head_dim, capacity * head_dim if stride is None else stride, capacity, max_batch,
                  int(r16), 0)
    rc = library().hsdpa_kv_check(ctypes.byref(spec))
    if rc != 0:
        raise HsdpaError(rc, "hsdpa_kv_check")
    return spec


def kv_append_raw(spec: KvSpec, keys: int, values: int, input_keys: int, input_values: int, rows: int,
                  past: int, stream: int = 0) -> None:
    call = KvCall(keys, values, input_keys, input_values, rows, past)
    rc = library().hsdpa_kv_append(ctypes.byref(spec), ctypes.byref(call), ctypes.c_void_p(stream))
    if rc != 0:
        raise HsdpaError(rc, "hsdpa_kv_append")


def kv_append_torch(spec: KvSpec, keys, values, input_keys, input_values, rows: int, past: int,
                    stream=None) -> None:
    """The kv-append node on torch device tensors holding bf16 bits. Views at
    any element offset are accepted (unaligned ones take the scalar path)."""
    import torch

    for t in (keys, values, input_keys, input_values):
        if not t.is_cuda:
            raise ValueError("tensors must be device tensors")
    s = torch.cuda.current_stream() if stream is None else stream
    kv_append_raw(spec, keys.data_ptr(), values.data_ptr(), input_keys.data_ptr(), input_values.data_ptr(),
                  rows, past, s.cuda_stream)


def head_norm_rope_torch(data, weight, cos, sin, heads: int, head_dim: int, head_stride: int, row_stride: int,
                         rotary_dims: int, rows: int, past: int, eps: float, plus_one: bool = True,
                         table_row: int | None = None, positions: int | None = None, stream=None) -> None:
    """The head-norm-rope node on torch device tensors holding bf16 bits; data
    is updated in place. cos/sin are [positions][table_row] tables."""
    import torch

    half = rotary_dims // 2
    tr = half if table_row is None else table_row
    pos = (cos.numel() // tr if tr else 0) if positions is None else positions
    spec = NormRopeSpec(heads, head_dim, head_stride, row_stride, rotary_dims, tr, pos, int(plus_one), 0)
    call = NormRopeCall(data.data_ptr(), weight.data_ptr(), cos.data_ptr() if cos is not None else 0,
                        sin.data_ptr() if sin is not None else 0, rows, past, eps, 0.0)
    s = torch.cuda.current_stream() if stream is None else stream
    rc = library().hsdpa_head_norm_rope(ctypes.byref(spec), ctypes.byref(call), ctypes.c_void_p(s.cuda_stream))
    if rc != 0:
        raise HsdpaError(rc, "hsdpa_head_norm_rope")


def output_gate_torch(attn, gate, width: int, attn_row: int, gate_row: int, rows: int, stream=None) -> None:
    """attn <- attn * sigmoid(gate) in place (torch device tensors of bf16 bits;
    `gate` may be a view starting at q + q_dim)."""
    import torch

    spec = GateSpec(width, attn_row, gate_row)
    call = GateCall(attn.data_ptr(), gate.data_ptr(), rows)
    s = torch.cuda.current_stream() if stream is None else stream
    rc = library().hsdpa_output_gate(ctypes.byref(spec), ctypes.byref(call), ctypes.c_void_p(s.cuda_stream))
    if rc != 0:
        raise HsdpaError(rc, "hsdpa_output_gate")


def kv_restore_raw(spec: KvSpec, snapshot_layer: int, snap_positions: int, keys: int, values: int,
                   positions: int, stream: int = 0) -> None:
    """Copy the leading `positions` of every head of one snapshot layer (host,
    K[heads][snap_positions][head_dim] then V) into the live cache (device)."""
    rc = library().hsdpa_kv_restore(ctypes.byref(spec), snapshot_layer, snap_positions, keys, values, positions,
                                    ctypes.c_void_p(stream))
    if rc != 0:
        raise HsdpaError(rc, "hsdpa_kv_restore")


def kv_take_raw(spec: KvSpec, keys: int, values: int, snapshot_layer: int, snap_positions: int, positions: int,
                stream: int = 0) -> None:
    """Copy the leading `positions` of every head of the live cache (device)
    into one snapshot layer (host)."""
    rc = library().hsdpa_kv_take(ctypes.byref(spec), keys, values, snapshot_layer, snap_positions, positions,
                                 ctypes.c_void_p(stream))
    if rc != 0:
        raise HsdpaError(rc, "hsdpa_kv_take")


def attention_layer_torch(plan: Plan, q, k, v, keys, values, out, q_norm, k_norm, cos, sin, rows: int, past: int,
                          scale: float, eps: float, workspace, kv_row: int, rotary_dims: int, gate=None,
                          gate_row: int = 0, plus_one: bool = True, table_row: int | None = None,
                          positions: int | None = None, stream=None) -> None:
    """The layer chain (hsdpa_attention_layer) on torch device tensors holding
    bf16 bits: q and k normalised and rotated in place, k and v appended to
    the cache at `past`, the attention into `out`, gated when `gate` (a view,
    e.g. of q at q_dim) is given."""
    import torch

    tr = rotary_dims // 2 if table_row is None else table_row
    pos = (cos.numel() // tr if tr else 0) if positions is None else positions
    ptr = lambda t: t.data_ptr() if t is not None else 0
    call = LayerCall(ptr(q), ptr(k), ptr(v), ptr(keys), ptr(values), ptr(out), ptr(gate), ptr(q_norm), ptr(k_norm),
                     ptr(cos), ptr(sin), rows, past, kv_row, gate_row, rotary_dims, tr, pos, scale, eps,
                     int(plus_one), 0, ptr(workspace), workspace.numel() * workspace.element_size())
    s = torch.cuda.current_stream() if stream is None else stream
    rc = library().hsdpa_attention_layer(plan.handle, ctypes.byref(call), ctypes.c_void_p(s.cuda_stream))
    if rc != 0:
        raise HsdpaError(rc, "hsdpa_attention_layer")
