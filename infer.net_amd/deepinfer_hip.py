"""Python binding of libdeepinfer_hip (the C ABI in include/deepinfer_hip.h).

Two layers:
  * ``QuantizedHip`` / ``QuantMatrix`` mirror the managed device of the reference,
    ``QuantizedMetal`` / ``QuantMatrix`` (src/DeepInfer.Backends/Compute/QuantizedMetal.cs):
    same methods, argument meaning, validation order and exception kinds, with host
    float32 numpy arrays in and out (synchronous).
  * module functions ``qmv``, ``qmv_swiglu``, ``lm_head``, ``argmax``, ``top8``,
    ``build_groups``, ``dequant_bf16``, ``moe_decode``, ``moe_prefill`` and ``dense`` take
    device tensors (anything with ``data_ptr()``) and enqueue work on the current torch
    stream (PyTorch is only used for device memory and streams).

The library is loaded from ``lib/libdeepinfer_hip.so`` next to this file; importing this
module fails loudly if it has not been built (there is no CPU fallback).
"""
from __future__ import annotations

import ctypes
import os
from typing import Optional, Sequence

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "lib", "libdeepinfer_hip.so")
HEADER_PATH = os.path.join(os.path.dirname(_HERE), "include", "deepinfer_hip.h")

F32, BF16 = 0, 1
_ERR = 2048


# Exception kinds of the managed reference (QuantizedMetal.cs / QuantizedTests.cs).
class ArgumentError(ValueError):
    """System.ArgumentException"""


class ArgumentOutOfRangeError(ArgumentError):
    """System.ArgumentOutOfRangeException"""


class ObjectDisposedError(RuntimeError):
    """System.ObjectDisposedException"""


class InvalidOperationError(RuntimeError):
    """System.InvalidOperationException"""


class InvalidDataError(ValueError):
    """System.IO.InvalidDataException (checkpoint and safetensors validation)"""


class NotSupportedError(Exception):
    """System.NotSupportedException (unsupported dtype, geometry or quantization)"""


class Job(ctypes.Structure):
    _fields_ = [("matrix", ctypes.c_void_p), ("input", ctypes.c_void_p),
                ("output", ctypes.c_void_p), ("experts", ctypes.c_void_p),
                ("count", ctypes.c_int32), ("batched", ctypes.c_int32)]


class MoeLayer(ctypes.Structure):
    _fields_ = [(n, ctypes.c_void_p) for n in ("router", "gate", "up", "down", "shared_gate",
                                                "shared_up", "shared_down", "shared_route")]


class MoeTrace(ctypes.Structure):
    _fields_ = [(n, ctypes.c_void_p) for n in ("logits", "ids", "probs", "expert_out", "status")]


class MoeMerge(ctypes.Structure):
    """dih_moe_merge: residual storage and the fused next-layer RMSNorm."""
    _fields_ = [("residual_f32", ctypes.c_int), ("norm_weight", ctypes.c_void_p), ("epsilon", ctypes.c_float),
                ("normed", ctypes.c_void_p), ("normed_f32", ctypes.c_int)]


EXPORTS = [
    "dih_quant_create", "dih_quant_create_configured", "dih_quant_destroy",
    "dih_quant_residency_bytes", "dih_quant_residency_prepare", "dih_quant_matrix_create",
    "dih_quant_matrix_buffer", "dih_quant_matrix_destroy", "dih_quant_matrix_write",
    "dih_quant_matrix_commit", "dih_quant_matrix_device", "dih_quant_matrix_shape",
    "dih_quant_batch", "dih_quant_matvec", "dih_quant_experts", "dih_quant_embedding",
    "dih_qmv", "dih_qmv_swiglu", "dih_lm_head", "dih_argmax", "dih_top8", "dih_build_groups",
    "dih_dequant_bf16", "dih_moe_decode", "dih_moe_prefill", "dih_moe_decode_norm", "dih_moe_decode_noalloc",
    "dih_moe_prefill_norm", "dih_grouped_qmm", "dih_dense", "dih_attention",
    "dih_attention_partition", "dih_delta_rule", "dih_delta_create", "dih_delta_destroy",
    "dih_delta_step", "dih_set_profiling",
    "dih_profile_read", "dih_version",
    "dih_safetensors_open", "dih_safetensors_close", "dih_safetensors_count",
    "dih_safetensors_info", "dih_safetensors_get", "dih_safetensors_read",
    "dih_safetensors_read_float", "dih_checkpoint_open", "dih_checkpoint_close",
    "dih_checkpoint_info", "dih_checkpoint_matrix", "dih_checkpoint_vector",
    "dih_checkpoint_moe_layer",
]

_lib = None


def load():
    """Loads the built library (raises OSError naming the missing file if absent)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise OSError(f"libdeepinfer_hip is not built: {LIB_PATH} missing "
                      "(run __graft_entry__.build() or make -C infer.net_amd)")
    L = ctypes.CDLL(LIB_PATH)
    P, I, S = ctypes.c_void_p, ctypes.c_int, ctypes.c_size_t
    E = ctypes.c_char_p
    sig = {
        "dih_quant_create": ([E, I], P),
        "dih_quant_create_configured": ([I, I, E, I], P),
        "dih_quant_destroy": ([P], None),
        "dih_quant_residency_bytes": ([P], ctypes.c_uint64),
        "dih_quant_residency_prepare": ([P], None),
        "dih_quant_matrix_create": ([P, I, I, I, I, I, E, I], P),
        "dih_quant_matrix_buffer": ([P, I], P),
        "dih_quant_matrix_destroy": ([P], None),
        "dih_quant_matrix_write": ([P, I, S, P, S, E, I], I),
        "dih_quant_matrix_commit": ([P, E, I], I),
        "dih_quant_matrix_device": ([P, I], P),
        "dih_quant_matrix_shape": ([P, P, P, P, P], I),
        "dih_quant_batch": ([P, P, I, P, E, I], I),
        "dih_quant_matvec": ([P, P, P, P, P, I, I, P, E, I], I),
        "dih_quant_experts": ([P, P, P, P, P, P, P, P, I, P, P, P, E, I], I),
        "dih_quant_embedding": ([P, I, P], I),
        "dih_qmv": ([P, P, P, I, P, I, P, I, I, P, E, I], I),
        "dih_qmv_swiglu": ([P, P, P, P, I, P, P, I, P, E, I], I),
        "dih_lm_head": ([P, P, I, P, P, P, P, E, I], I),
        "dih_argmax": ([P, P, I, P, P, E, I], I),
        "dih_top8": ([P, P, I, I, I, P, P, P, P, E, I], I),
        "dih_build_groups": ([P, P, I, I, P, P, P, E, I], I),
        "dih_dequant_bf16": ([P, P, I, P, P, E, I], I),
        "dih_moe_decode": ([P, P, P, P, P, P, P, E, I], I),
        "dih_moe_prefill": ([P, P, I, P, P, I, P, P, P, E, I], I),
        "dih_moe_decode_norm": ([P, P, P, P, P, P, P, P, E, I], I),
        "dih_moe_decode_noalloc": ([P, P, P, P, P, P, P, P, E, I], I),
        "dih_moe_prefill_norm": ([P, P, I, P, P, I, P, P, P, P, E, I], I),
        "dih_dense": ([P, P, I, P, P, I, P, E, I], I),
        "dih_grouped_qmm": ([P, P, P, I, P, I, P, P, P, I, P, E, I], I),
        "dih_attention": ([P, P, I, P, P, I, P, I, P, I, I, I, I, P, E, I], I),
        "dih_attention_partition": ([I, I, I], I),
        "dih_delta_rule": ([P, P, P, P, P, P, P, P, I, I, P, E, I], I),
        "dih_delta_create": ([P], P),
        "dih_delta_destroy": ([P], None),
        "dih_delta_step": ([P, P, P, P, P, P, P, P, P, E, I], I),
        "dih_set_profiling": ([P, I], I),
        "dih_profile_read": ([P, P, P, P, I], I),
        "dih_version": ([], ctypes.c_char_p),
        "dih_safetensors_open": ([E, P, E, I], P),
        "dih_safetensors_close": ([P], None),
        "dih_safetensors_count": ([P], I),
        "dih_safetensors_info": ([P, I, E, I, P, P, P, P], I),
        "dih_safetensors_get": ([P, E, P, I, E, I], I),
        "dih_safetensors_read": ([P, E, I, P, ctypes.c_uint64, E, I], I),
        "dih_safetensors_read_float": ([P, E, P, ctypes.c_uint64, E, I], I),
        "dih_checkpoint_open": ([E, P, E, I], P),
        "dih_checkpoint_close": ([P], None),
        "dih_checkpoint_info": ([P, P, P, P], I),
        "dih_checkpoint_matrix": ([P, P, E, I, I, I, I, P, E, I], P),
        "dih_checkpoint_vector": ([P, E, P, I, P, ctypes.c_uint64, E, I], I),
        "dih_checkpoint_moe_layer": ([P, P, I, P, E, I], I),
    }
    for name, (args, res) in sig.items():
        fn = getattr(L, name)
        fn.argtypes = args
        fn.restype = res
    _lib = L
    return L


def _errbuf():
    return ctypes.create_string_buffer(_ERR)


def _msg(buf) -> str:
    return buf.value.decode("utf-8", "replace")


def _check(rc, buf, kind=InvalidOperationError):
    if rc != 0:
        raise kind(_msg(buf))


def _dp(t) -> Optional[int]:
    """Device pointer of a tensor-like (data_ptr()) or an int; None passes NULL."""
    if t is None:
        return None
    if isinstance(t, int):
        return t
    return t.data_ptr()


def _stream(stream) -> Optional[int]:
    """The stream handle to pass: an explicit stream, else torch's current stream. Torch's
    default stream is the HIP null stream (handle 0): it goes as NULL, which selects the
    context's blocking stream, ordered against the null stream in both directions."""
    if stream is not None:
        return stream if isinstance(stream, int) else stream.cuda_stream
    try:
        import torch
        return torch.cuda.current_stream().cuda_stream
    except Exception:  # pragma: no cover - torch without a device
        return None


class QuantizedHip:
    """Mirror of ``QuantizedMetal`` (QuantizedMetal.cs:7-146) over the HIP C ABI."""

    def __init__(self, batch_submissions: bool = True, residency: Optional[bool] = None,
                 residency_refresh_milliseconds: int = 1000):
        if not 0 <= residency_refresh_milliseconds <= 60000:
            raise ArgumentOutOfRangeError("residencyRefreshMilliseconds")
        self.batch_submissions = batch_submissions
        self.dispatches = 0
        self.submissions = 0
        self.gpu_milliseconds = 0.0
        L = load()
        err = _errbuf()
        if residency is None:
            p = L.dih_quant_create(err, _ERR)
        else:
            p = L.dih_quant_create_configured(1 if residency else 0, residency_refresh_milliseconds, err, _ERR)
        if not p:
            raise InvalidOperationError(_msg(err))
        self.context = p
        self._lib = L

    # QuantizedMetal.cs:30-31
    @property
    def residency_bytes(self) -> int:
        self._alive()
        return int(self._lib.dih_quant_residency_bytes(self.context))

    def prepare_residency(self) -> None:
        self._alive()
        self._lib.dih_quant_residency_prepare(self.context)

    def _alive(self):
        if self.context is None:
            raise ObjectDisposedError("QuantizedHip")

    def allocate(self, experts: int, rows: int, columns: int, bits: int, group: int = 64) -> "QuantMatrix":
        """QuantizedMetal.Allocate (QuantizedMetal.cs:32-46)."""
        self._alive()
        if (not 1 <= experts <= 256 or not 1 <= rows <= 262144 or not 64 <= columns <= 32768
                or columns % 64 != 0 or bits not in (5, 8) or group != 64):
            raise ArgumentError("Unsupported quantized shape/precision.")
        if experts * rows * (columns * bits // 8) > 2**63 - 1:
            raise OverflowError()
        err = _errbuf()
        p = self._lib.dih_quant_matrix_create(self.context, experts, rows, columns, bits, group, err, _ERR)
        if not p:
            raise InvalidOperationError(_msg(err))
        return QuantMatrix(self, p, experts, rows, columns, bits)

    def new_delta_memory(self) -> "DeltaMemory":
        """QuantizedMetal.NewDeltaMemory (QuantizedMetal.cs:47-52)."""
        self._alive()
        p = self._lib.dih_delta_create(self.context)
        if not p:
            raise InvalidOperationError("Cannot allocate gated-delta state.")
        return DeltaMemory(self, p)

    def multiply_batch(self, jobs: Sequence["QuantizedJob"]) -> None:
        """QuantizedMetal.MultiplyBatch (QuantizedMetal.cs:54-112): 1..8 independent jobs."""
        self._alive()
        if not 1 <= len(jobs) <= 8:
            raise ArgumentError("Expected 1..8 independent GEMV jobs.")
        for i, job in enumerate(jobs):
            if job.matrix is None or job.input is None or job.output is None:
                raise ArgumentError("Incomplete GEMV job.")
            if job.matrix.owner is not self:
                raise ArgumentError("Batch matrices must belong to this device.")
            job.matrix.validate(len(job.input), len(job.output), job.experts if job.experts is not None else [0],
                                job.batched)
            for prev in jobs[:i]:
                if (job.matrix is prev.matrix or job.output is prev.output or job.output is prev.input
                        or job.input is prev.output):
                    raise ArgumentError("GEMV jobs must have distinct matrices/outputs and no cross-job dependencies.")
        if not self.batch_submissions:
            for job in jobs:
                job.matrix.multiply_experts(job.input, job.output, job.experts if job.experts is not None else [0],
                                            job.batched)
            return
        natives = (Job * len(jobs))()
        keep = []
        for i, job in enumerate(jobs):
            x = _f32_in(job.input)
            y = _f32_out(job.output)
            ids = np.ascontiguousarray(job.experts if job.experts is not None else [0], dtype=np.uint32)
            keep += [x, y, ids]
            natives[i] = Job(job.matrix.handle, x.ctypes.data, y.ctypes.data, ids.ctypes.data, len(ids),
                             1 if job.batched else 0)
        err = _errbuf()
        ms = ctypes.c_double()
        rc = self._lib.dih_quant_batch(self.context, natives, len(jobs), ctypes.byref(ms), err, _ERR)
        _check(rc, err)
        for k, job in enumerate(jobs):
            _copy_back(keep[3 * k + 1], job.output)
        self.count(ms.value, len(jobs))

    def expert_mlp(self, gate, up, down, shared_down, input, shared_input, experts, expert_output,
                   shared_output) -> None:
        """QuantizedMetal.ExpertMlp (QuantizedMetal.cs:115-142)."""
        self._alive()
        mats = [gate, up, down, shared_down]
        for i, m in enumerate(mats):
            if m is None or m.owner is not self:
                raise ArgumentError("Expert matrices must belong to this device.")
            for prev in mats[:i]:
                if m is prev:
                    raise ArgumentError("Expert matrices must be distinct.")
        if (gate.rows != up.rows or gate.columns != up.columns or gate.experts != up.experts or gate.bits != up.bits
                or down.columns != gate.rows or down.rows != gate.columns or down.experts != gate.experts
                or shared_down.experts != 1 or shared_down.rows != down.rows
                or _overlaps(expert_output, shared_output)):
            raise ArgumentError("Incompatible expert shapes/precision or overlapping outputs.")
        gate.validate(len(input), gate.rows * len(experts), experts, False)
        up.validate(len(input), up.rows * len(experts), experts, False)
        down.validate(gate.rows * len(experts), len(expert_output), experts, True)
        shared_down.validate(len(shared_input), len(shared_output), [0], False)
        x = _f32_in(input)
        sx = _f32_in(shared_input)
        ids = np.ascontiguousarray(experts, dtype=np.uint32)
        y = _f32_out(expert_output)
        sy = _f32_out(shared_output)
        err = _errbuf()
        ms = ctypes.c_double()
        rc = self._lib.dih_quant_experts(self.context, gate.handle, up.handle, down.handle, shared_down.handle,
                                         x.ctypes.data, sx.ctypes.data, ids.ctypes.data, len(ids), y.ctypes.data,
                                         sy.ctypes.data, ctypes.byref(ms), err, _ERR)
        _check(rc, err)
        _copy_back(y, expert_output)
        _copy_back(sy, shared_output)
        self.count(ms.value, 3)

    def count(self, ms: float, dispatches: int = 1, submissions: int = 1) -> None:
        self.dispatches += dispatches
        self.submissions += submissions
        self.gpu_milliseconds += ms

    def dispose(self) -> None:
        if self.context is not None:
            self._lib.dih_quant_destroy(self.context)
            self.context = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.dispose()


class QuantizedJob:
    """QuantizedJob record (QuantizedMetal.cs:146)."""

    def __init__(self, matrix, input, output, experts=None, batched=False):
        self.matrix, self.input, self.output = matrix, input, output
        self.experts, self.batched = experts, batched


class QuantMatrix:
    """Mirror of ``QuantMatrix`` (QuantizedMetal.cs:148-205)."""

    def __init__(self, owner: QuantizedHip, handle, experts, rows, columns, bits):
        self.owner, self.handle = owner, handle
        self.experts, self.rows, self.columns, self.bits = experts, rows, columns, bits

    def _alive(self):
        if self.handle is None or self.owner.context is None:
            raise ObjectDisposedError("QuantMatrix")

    def buffer_bytes(self, index: int) -> int:
        if not 0 <= index <= 2:
            raise ArgumentOutOfRangeError("index")
        per = self.columns * self.bits // 8 if index == 0 else self.columns // 64 * 2
        return self.experts * self.rows * per

    def write(self, index: int, data) -> None:
        """QuantMatrix.Write (QuantizedMetal.cs:171-176) through the host staging pointer
        (dih_quant_matrix_buffer), uploaded before the next GPU use."""
        self._alive()
        raw = np.ascontiguousarray(data).view(np.uint8).reshape(-1)
        if raw.size != self.buffer_bytes(index):
            raise ArgumentError("Quantized buffer length mismatch.")
        p = self.owner._lib.dih_quant_matrix_buffer(self.handle, index)
        if not p:
            raise InvalidOperationError("Missing quantized buffer.")
        ctypes.memmove(p, raw.ctypes.data, raw.size)

    def upload(self, index: int, data, offset: int = 0) -> None:
        """Direct device upload without a host staging copy (dih_quant_matrix_write)."""
        self._alive()
        raw = np.ascontiguousarray(data).view(np.uint8).reshape(-1)
        err = _errbuf()
        _check(self.owner._lib.dih_quant_matrix_write(self.handle, index, offset, raw.ctypes.data, raw.size, err,
                                                      _ERR), err, ArgumentError)

    def upload_from(self, index: int, tensor, offset: int = 0) -> None:
        """Copies a device (or host) tensor's bytes into buffer `index`."""
        self._alive()
        nbytes = tensor.numel() * tensor.element_size()
        err = _errbuf()
        _check(self.owner._lib.dih_quant_matrix_write(self.handle, index, offset, tensor.data_ptr(), nbytes, err,
                                                      _ERR), err, ArgumentError)

    def device_ptr(self, index: int) -> int:
        self._alive()
        p = self.owner._lib.dih_quant_matrix_device(self.handle, index)
        if not p:
            raise InvalidOperationError("Missing device buffer.")
        return p

    def multiply(self, input, output) -> None:
        self.multiply_experts(input, output, [0])

    def multiply_experts(self, input, output, experts, batched: bool = False) -> None:
        """QuantMatrix.MultiplyExperts (QuantizedMetal.cs:180-191)."""
        self.validate(len(input), len(output), experts, batched)
        x = _f32_in(input)
        y = _f32_out(output)
        ids = np.ascontiguousarray(experts, dtype=np.uint32)
        err = _errbuf()
        ms = ctypes.c_double()
        rc = self.owner._lib.dih_quant_matvec(self.owner.context, self.handle, x.ctypes.data, y.ctypes.data,
                                              ids.ctypes.data, len(ids), 1 if batched else 0, ctypes.byref(ms),
                                              err, _ERR)
        _check(rc, err)
        _copy_back(y, output)
        self.owner.count(ms.value)

    def validate(self, input_length: int, output_length: int, experts, batched: bool) -> None:
        """QuantMatrix.Validate (QuantizedMetal.cs:192-198)."""
        self._alive()
        n = len(experts)
        if not 1 <= n <= 8 or input_length != self.columns * (n if batched else 1) or output_length != self.rows * n:
            raise ArgumentError("Quantized GEMV input/output shape mismatch.")
        for e in experts:
            if e < 0 or e >= self.experts:
                raise ArgumentOutOfRangeError("experts")

    def copy_row(self, token: int, output) -> None:
        """QuantMatrix.CopyRow (QuantizedMetal.cs:199-205)."""
        self._alive()
        if len(output) != self.columns or token < 0 or token >= self.rows or self.experts != 1:
            raise ArgumentError("Invalid embedding row.")
        y = _f32_out(output)
        if self.owner._lib.dih_quant_embedding(self.handle, token, y.ctypes.data) != 0:
            raise InvalidOperationError("Embedding lookup failed.")
        _copy_back(y, output)

    def dispose(self) -> None:
        if self.handle is not None:
            self.owner._lib.dih_quant_matrix_destroy(self.handle)
            self.handle = None


class DeltaMemory:
    """Mirror of ``DeltaMemory`` (QuantizedMetal.cs:207-225): one linear-attention layer's
    recurrent state on the device, stepped one token at a time from host arrays."""

    def __init__(self, owner: QuantizedHip, handle):
        self.owner, self.handle = owner, handle

    def step(self, q, k, v, decay, beta, output) -> None:
        """DeltaMemory.Step (QuantizedMetal.cs:212-225)."""
        if self.handle is None or self.owner.context is None:
            raise ObjectDisposedError("DeltaMemory")
        if (len(q) != 2048 or len(k) != 2048 or len(v) != 4096 or len(decay) != 32 or len(beta) != 32
                or len(output) != 4096):
            raise ArgumentError("Unsupported gated-delta dimensions.")
        qa, ka, va, ga, ba = (_f32_in(a) for a in (q, k, v, decay, beta))
        y = _f32_out(output)
        err = _errbuf()
        ms = ctypes.c_double()
        rc = self.owner._lib.dih_delta_step(self.owner.context, self.handle, qa.ctypes.data, ka.ctypes.data,
                                            va.ctypes.data, ga.ctypes.data, ba.ctypes.data, y.ctypes.data,
                                            ctypes.byref(ms), err, _ERR)
        _check(rc, err)
        _copy_back(y, output)
        self.owner.count(ms.value)

    def dispose(self) -> None:
        if self.handle is not None:
            self.owner._lib.dih_delta_destroy(self.handle)
            self.handle = None


def _f32_in(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def _f32_out(a) -> np.ndarray:
    if isinstance(a, np.ndarray) and a.dtype == np.float32 and a.flags.c_contiguous:
        return a
    return np.zeros(len(a), dtype=np.float32)


def _copy_back(src: np.ndarray, dst) -> None:
    if src is not dst:
        dst[:] = src


def _overlaps(a, b) -> bool:
    if isinstance(a, np.ndarray) and isinstance(b, np.ndarray):
        return np.shares_memory(a, b)
    return a is b


# ------------------------------------------------------------------ device-resident ops

def _ctx(dev: QuantizedHip):
    dev._alive()
    return dev.context


def qmv(dev: QuantizedHip, m: QuantMatrix, x, y, experts=None, count: int = 1, batched: bool = False,
        x_dtype: int = BF16, y_dtype: int = F32, stream=None) -> None:
    err = _errbuf()
    _check(dev._lib.dih_qmv(_ctx(dev), m.handle, _dp(x), x_dtype, _dp(y), y_dtype, _dp(experts), count,
                            1 if batched else 0, _stream(stream), err, _ERR), err, ArgumentError)


def qmv_swiglu(dev, gate, up, x, act, experts=None, count=1, x_dtype=BF16, stream=None) -> None:
    err = _errbuf()
    _check(dev._lib.dih_qmv_swiglu(_ctx(dev), gate.handle, up.handle, _dp(x), x_dtype, _dp(act), _dp(experts),
                                   count, _stream(stream), err, _ERR), err, ArgumentError)


def lm_head(dev, slices, x, logits, next_token, stream=None) -> None:
    arr = (ctypes.c_void_p * len(slices))(*[s.handle for s in slices])
    err = _errbuf()
    _check(dev._lib.dih_lm_head(_ctx(dev), arr, len(slices), _dp(x), _dp(logits), _dp(next_token),
                                _stream(stream), err, _ERR), err, ArgumentError)


def argmax(dev, values, n, next_token, stream=None) -> None:
    err = _errbuf()
    _check(dev._lib.dih_argmax(_ctx(dev), _dp(values), n, _dp(next_token), _stream(stream), err, _ERR), err,
           ArgumentError)


def top8(dev, logits, tokens, experts, ids, probs, status=None, logits_dtype=BF16, stream=None) -> None:
    err = _errbuf()
    _check(dev._lib.dih_top8(_ctx(dev), _dp(logits), logits_dtype, tokens, experts, _dp(ids), _dp(probs),
                             _dp(status), _stream(stream), err, _ERR), err, ArgumentError)


def build_groups(dev, ids, tokens, experts, counts, routes, stream=None) -> None:
    err = _errbuf()
    _check(dev._lib.dih_build_groups(_ctx(dev), _dp(ids), tokens, experts, _dp(counts), _dp(routes),
                                     _stream(stream), err, _ERR), err, ArgumentError)


def dequant_bf16(dev, m, expert, out, stream=None) -> None:
    err = _errbuf()
    _check(dev._lib.dih_dequant_bf16(_ctx(dev), m.handle, expert, _dp(out), _stream(stream), err, _ERR), err,
           ArgumentError)


def make_layer(router, gate, up, down, shared_gate, shared_up, shared_down, shared_route) -> MoeLayer:
    h = lambda m: None if m is None else m.handle  # noqa: E731
    return MoeLayer(h(router), h(gate), h(up), h(down), h(shared_gate), h(shared_up), h(shared_down),
                    h(shared_route))


def make_trace(logits=None, ids=None, probs=None, expert_out=None, status=None) -> MoeTrace:
    return MoeTrace(_dp(logits), _dp(ids), _dp(probs), _dp(expert_out), _dp(status))


def make_merge(residual_f32=False, norm_weight=None, epsilon=1e-6, normed=None, normed_f32=True) -> MoeMerge:
    return MoeMerge(1 if residual_f32 else 0, _dp(norm_weight), epsilon, _dp(normed), 1 if normed_f32 else 0)


def moe_decode(dev, layer: MoeLayer, x, residual, logits=None, trace: Optional[MoeTrace] = None,
               stream=None, merge: Optional[MoeMerge] = None) -> None:
    err = _errbuf()
    _check(dev._lib.dih_moe_decode_norm(_ctx(dev), ctypes.byref(layer), _dp(x), _dp(logits), _dp(residual),
                                        None if merge is None else ctypes.byref(merge),
                                        None if trace is None else ctypes.byref(trace), _stream(stream), err, _ERR),
           err, ArgumentError)


def moe_decode_noalloc(dev, layer: MoeLayer, x, residual, logits=None, trace: Optional[MoeTrace] = None,
                       stream=None, merge: Optional[MoeMerge] = None) -> None:
    """moe_decode without any device allocation (dih_moe_decode_noalloc): intermediates live
    in the library's fixed per-GPU scratch array; overlapping calls on one GPU race."""
    err = _errbuf()
    _check(dev._lib.dih_moe_decode_noalloc(_ctx(dev), ctypes.byref(layer), _dp(x), _dp(logits), _dp(residual),
                                           None if merge is None else ctypes.byref(merge),
                                           None if trace is None else ctypes.byref(trace), _stream(stream), err,
                                           _ERR), err, ArgumentError)


def moe_prefill(dev, layer: MoeLayer, tokens, x, logits, residual, logits_dtype=BF16,
                trace: Optional[MoeTrace] = None, stream=None, merge: Optional[MoeMerge] = None) -> None:
    err = _errbuf()
    _check(dev._lib.dih_moe_prefill_norm(_ctx(dev), ctypes.byref(layer), tokens, _dp(x), _dp(logits),
                                         logits_dtype, _dp(residual), None if merge is None else ctypes.byref(merge),
                                         None if trace is None else ctypes.byref(trace), _stream(stream), err,
                                         _ERR), err, ArgumentError)


def grouped_qmm(dev, m, tokens, x, counts, routes, y, up=None, input_mode=0, y_dtype=F32, stream=None) -> None:
    """One grouped expert projection over dih_build_groups route lists (dih_grouped_qmm):
    gate/up + SwiGLU when `up` is given (input_mode 1: token rows), else a plain grouped
    product (input_mode 0: route rows)."""
    err = _errbuf()
    _check(dev._lib.dih_grouped_qmm(_ctx(dev), m.handle, None if up is None else up.handle, tokens, _dp(x),
                                    input_mode, _dp(counts), _dp(routes), _dp(y), y_dtype, _stream(stream), err,
                                    _ERR), err, ArgumentError)


def dense(dev, m, tokens, x, y, y_dtype=F32, stream=None) -> None:
    err = _errbuf()
    _check(dev._lib.dih_dense(_ctx(dev), m.handle, tokens, _dp(x), _dp(y), y_dtype, _stream(stream), err, _ERR),
           err, ArgumentError)


def attention(dev, q, keys, values, gate, out, position, tokens, partition=0, q_dtype=F32,
              gate_dtype=F32, out_dtype=F32, cache_positions=None, stream=None) -> None:
    """Causal GQA attention with the output gate (dih_attention; p_fused_attention,
    gpu_prefill.mm:552-570). keys/values: bf16 cache tensors [cache_positions, 512].
    partition: the rounding partition (0: the reference's 1024; 32: every 32-key block its
    own partition, the fastest decode form)."""
    if cache_positions is None:
        cache_positions = keys.shape[0]
    err = _errbuf()
    _check(dev._lib.dih_attention(_ctx(dev), _dp(q), q_dtype, _dp(keys), _dp(values), cache_positions,
                                  _dp(gate), gate_dtype, _dp(out), out_dtype, position, tokens, partition,
                                  _stream(stream), err, _ERR), err, ArgumentError)


def delta_rule(dev, state, history, conv, decay, beta, raw, out, tokens, path=0, stream=None) -> None:
    """Gated delta rule over a chunk (dih_delta_rule; p_delta, gpu_prefill.mm:540-551).
    path 0: chunkwise from 64 tokens, sequential below (the library's choice); 1:
    sequential; 2: chunkwise."""
    err = _errbuf()
    _check(dev._lib.dih_delta_rule(_ctx(dev), _dp(state), _dp(history), _dp(conv), _dp(decay), _dp(beta),
                                   _dp(raw), _dp(out), tokens, path, _stream(stream), err, _ERR),
           err, ArgumentError)


def attention_partition(position, tokens, partition=0) -> int:
    """Rounding partition dih_attention uses for these arguments (1024 unless given)."""
    n = load().dih_attention_partition(position, tokens, partition)
    if n < 0:
        raise ArgumentError("Invalid attention arguments")
    return n


def set_profiling(dev, enabled: bool) -> None:
    dev._lib.dih_set_profiling(_ctx(dev), 1 if enabled else 0)


def profile_read(dev):
    """{stage name: (total ms, launches)} recorded since set_profiling(dev, True)."""
    ms = (ctypes.c_double * 32)()
    counts = (ctypes.c_int * 32)()
    names = (ctypes.c_char_p * 32)()
    n = dev._lib.dih_profile_read(_ctx(dev), ms, counts, names, 32)
    if n < 0:
        raise InvalidOperationError("profile read failed")
    return {names[i].decode(): (ms[i], counts[i]) for i in range(n)}


# ---------------------------------------------------------------------------------------
# Checkpoint loading: SafeTensors (SafeTensors.cs) and the MLX checkpoint directory
# (Qwen36Weights.cs), backed by the library's native reader and uploader.

_DTYPES = {1: "BF16", 2: "F32", 3: "U32"}


def _st_raise(code, buf):
    if code == -2:
        raise NotSupportedError(_msg(buf))
    raise InvalidDataError(_msg(buf))


def _enc(s: str) -> bytes:
    return s.encode("utf-8")


class SafeTensors:
    """Mirror of SafeTensors (SafeTensors.cs:7-95): a validated header and typed reads."""

    class Tensor:
        __slots__ = ("name", "dtype", "shape", "bytes", "_owner")

        def __init__(self, name, dtype, shape, nbytes, owner):
            self.name, self.dtype, self.shape, self.bytes, self._owner = name, dtype, tuple(shape), nbytes, owner

        def __repr__(self):
            return f"Tensor({self.name!r}, {self.dtype}, {list(self.shape)}, {self.bytes})"

    def __init__(self, path: str):
        L = load()
        err, st = _errbuf(), ctypes.c_int(0)
        h = L.dih_safetensors_open(_enc(os.fspath(path)), ctypes.byref(st), err, _ERR)
        if not h:
            _st_raise(st.value, err)
        self._h = h
        self._tensors = {}
        name = ctypes.create_string_buffer(4096)
        dt, rank = ctypes.c_int(), ctypes.c_int()
        shape = (ctypes.c_int64 * 8)()
        nbytes = ctypes.c_uint64()
        for i in range(L.dih_safetensors_count(h)):
            if L.dih_safetensors_info(h, i, name, 4096, ctypes.byref(dt), ctypes.byref(rank), shape,
                                      ctypes.byref(nbytes)) != 0:
                raise InvalidDataError("Invalid tensor entry.")
            n = name.value.decode("utf-8")
            self._tensors[n] = SafeTensors.Tensor(n, _DTYPES[dt.value], list(shape[:rank.value]),
                                                  nbytes.value, self)

    def _alive(self):
        if not self._h:
            raise ObjectDisposedError("SafeTensors")

    @property
    def tensors(self):
        return dict(self._tensors)

    def get(self, name: str, *shape: int) -> "SafeTensors.Tensor":
        self._alive()
        err = _errbuf()
        arr = (ctypes.c_int64 * max(1, len(shape)))(*shape)
        rc = load().dih_safetensors_get(self._h, _enc(name), arr, len(shape), err, _ERR)
        if rc != 0:
            _st_raise(rc, err)
        return self._tensors[name]

    def _own(self, tensor):
        if not isinstance(tensor, SafeTensors.Tensor) or tensor._owner is not self:
            raise InvalidDataError("Tensor ownership or destination length mismatch.")

    def read_into(self, tensor: "SafeTensors.Tensor", destination: np.ndarray) -> None:
        self._alive()
        self._own(tensor)
        if not (isinstance(destination, np.ndarray) and destination.flags.c_contiguous):
            raise InvalidDataError("Tensor ownership or destination length mismatch.")
        err = _errbuf()
        rc = load().dih_safetensors_read(self._h, _enc(tensor.name), 0, destination.ctypes.data,
                                         destination.nbytes, err, _ERR)
        if rc != 0:
            _st_raise(rc, err)

    def read_bfloat16(self, tensor: "SafeTensors.Tensor") -> np.ndarray:
        self._alive()
        self._own(tensor)
        out = np.empty(tensor.bytes // 2, dtype=np.uint16)
        err = _errbuf()
        rc = load().dih_safetensors_read(self._h, _enc(tensor.name), 1, out.ctypes.data, out.nbytes, err, _ERR)
        if rc != 0:
            _st_raise(rc, err)
        return out

    def read_float(self, tensor: "SafeTensors.Tensor") -> np.ndarray:
        self._alive()
        self._own(tensor)
        n = tensor.bytes // (2 if tensor.dtype == "BF16" else 4)
        out = np.empty(n, dtype=np.float32)
        err = _errbuf()
        rc = load().dih_safetensors_read_float(self._h, _enc(tensor.name), out.ctypes.data, n, err, _ERR)
        if rc != 0:
            _st_raise(rc, err)
        return out

    def dispose(self) -> None:
        if self._h:
            load().dih_safetensors_close(self._h)
            self._h = None

    close = dispose

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.dispose()


class Checkpoint:
    """The MLX checkpoint directory of Qwen36Weights (Qwen36Weights.cs:26-122): validated
    config, shard index, and matrices loaded straight into device memory."""

    def __init__(self, directory: str):
        L = load()
        err, st = _errbuf(), ctypes.c_int(0)
        h = L.dih_checkpoint_open(_enc(os.fspath(directory)), ctypes.byref(st), err, _ERR)
        if not h:
            _st_raise(st.value, err)
        self._h = h
        bits, eps, theta = ctypes.c_int(), ctypes.c_float(), ctypes.c_float()
        L.dih_checkpoint_info(h, ctypes.byref(bits), ctypes.byref(eps), ctypes.byref(theta))
        self.weight_bits, self.epsilon, self.rope_theta = bits.value, eps.value, theta.value

    def _alive(self):
        if not self._h:
            raise ObjectDisposedError("Checkpoint")

    def matrix(self, device: QuantizedHip, prefix: str, rows: int, columns: int, experts: int = 1,
               bits: int = 0) -> QuantMatrix:
        """Qwen36Weights.Matrix: PREFIX.{weight,scales,biases} -> a device-resident matrix."""
        self._alive()
        device._alive()
        err, st = _errbuf(), ctypes.c_int(0)
        h = load().dih_checkpoint_matrix(self._h, device.context, _enc(prefix), rows, columns, experts, bits,
                                         ctypes.byref(st), err, _ERR)
        if not h:
            _st_raise(st.value, err)
        return QuantMatrix(device, h, experts, rows, columns, bits or self.weight_bits)

    def vector(self, name: str, *shape: int) -> np.ndarray:
        """Qwen36Weights.Vector: ReadFloat of a tensor of exactly `shape`."""
        self._alive()
        n = int(np.prod(shape)) if shape else 0
        out = np.empty(n, dtype=np.float32)
        err = _errbuf()
        arr = (ctypes.c_int64 * max(1, len(shape)))(*shape)
        rc = load().dih_checkpoint_vector(self._h, _enc(name), arr, len(shape), out.ctypes.data, n, err, _ERR)
        if rc != 0:
            _st_raise(rc, err)
        return out

    def moe_layer(self, device: QuantizedHip, layer: int):
        """The eight MoE matrices of decoder layer `layer` (Qwen36Weights.cs:90-99); returns
        (MoeLayer for moe_decode/moe_prefill, [QuantMatrix] owning them)."""
        self._alive()
        device._alive()
        out, err = MoeLayer(), _errbuf()
        rc = load().dih_checkpoint_moe_layer(self._h, device.context, layer, ctypes.byref(out), err, _ERR)
        if rc != 0:
            _st_raise(rc, err)
        b = self.weight_bits
        shapes = [(256, 2048, 1, 8), (512, 2048, 256, b), (512, 2048, 256, b), (2048, 512, 256, b),
                  (512, 2048, 1, b), (512, 2048, 1, b), (2048, 512, 1, b), (1, 2048, 1, 8)]
        handles = [out.router, out.gate, out.up, out.down, out.shared_gate, out.shared_up,
                   out.shared_down, out.shared_route]
        mats = [QuantMatrix(device, h, e, r, c, bb) for h, (r, c, e, bb) in zip(handles, shapes)]
        return out, mats

    def dispose(self) -> None:
        if self._h:
            load().dih_checkpoint_close(self._h)
            self._h = None

    close = dispose

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.dispose()


def version() -> str:
    return load().dih_version().decode()
