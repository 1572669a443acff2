"""satori_amd: MI355X (gfx950) backend for Satori's quantized MatVec hot path.

Host-side mirror of the reference's surfaces over the C ABI of libsatori_hip.so (include/satori_hip.h).
Names, argument meaning and exceptions follow the reference (src/Satori.Core, src/Satori.Formats.Gguf):

  Ternary2Matrix.quantize / from_packed              Ternary2Matrix.cs:38-101
  Ternary2MatVec.execute                              Ternary2MatVec.cs:9 (HIP backend)
  MappedTernary2Matrix(path).execute                  MappedTernary2Matrix.cs:9-56 (HIP backend)
  QuantizedMatrixShape, BlockQuantization             QuantizedMatrixShape.cs:5-33, BlockQuantization.cs:3
  QuantizedMatVec.validate_payload / execute / execute_batch   QuantizedMatVec.cs:12-120 (HIP backend)
  HipContext.create(payload, shape)                   IQuantizedMatrixFactory.Create (IQuantizedMatrixFactory.cs:6)
  HipQuantizedMatrix.execute                          IQuantizedMatrix.Execute (IQuantizedMatrix.cs:7)
  Q8KCodec.quantize_row                               Q8KCodec.cs:85-93 (on the device)

Every MatVec runs on the GPU through the library; there is no CPU fallback. Importing this package needs
the built library (``python -m satori_amd.build``); creating a HipContext needs a gfx950 device.
"""
from __future__ import annotations

import ctypes
import enum
import os
import threading

import numpy as np

from . import _ffi

__all__ = [
    "SatoriError", "ArgumentException", "ArgumentOutOfRangeException", "ArgumentNullException",
    "InvalidDataException", "NotSupportedException", "ObjectDisposedException", "PlatformNotSupportedException",
    "OutOfMemoryException", "InvalidOperationException", "OverflowException", "KeyNotFoundException",
    "BlockQuantization", "QuantizedMatrixShape", "Ternary2Matrix", "Ternary2MatVec", "MappedTernary2Matrix",
    "QuantizedMatVec", "HipContext", "HipQuantizedMatrix", "HipGroup", "HipStep", "Q8KCodec", "TERNARY2",
    "device_count", "default_context", "payload_length", "quantize_weights",
    "GgufFile", "GgufTensor", "GgufMetadata", "GgufQuantizedMatrix", "GgufWeightStore",
    "TernaryBitplaneMatrix", "TernaryBitplaneMatVec", "TransformerOps", "DeviceOps",
]

TERNARY2 = 16


# ---- exceptions: one class per status code, named after the reference's .NET exception ----

class SatoriError(Exception):
    status = -1

    def __init__(self, message: str = ""):
        super().__init__(message)
        self.message = message


class ArgumentException(SatoriError, ValueError):
    status = 1


class ArgumentOutOfRangeException(ArgumentException):
    status = 2


class InvalidDataException(SatoriError, IOError):
    status = 3


class NotSupportedException(SatoriError):
    status = 4


class ObjectDisposedException(SatoriError):
    status = 5


class PlatformNotSupportedException(NotSupportedException):
    status = 6


class OutOfMemoryException(SatoriError, MemoryError):
    status = 7


class InvalidOperationException(SatoriError):
    status = 8


class OverflowException(SatoriError, ArithmeticError):
    status = 9


class ArgumentNullException(ArgumentException):
    status = 10


class KeyNotFoundException(SatoriError, KeyError):
    status = 11

    def __str__(self) -> str:  # KeyError would quote the message
        return self.message


_BY_STATUS = {cls.status: cls for cls in (
    ArgumentException, ArgumentOutOfRangeException, InvalidDataException, NotSupportedException,
    ObjectDisposedException, PlatformNotSupportedException, OutOfMemoryException, InvalidOperationException,
    OverflowException, ArgumentNullException, KeyNotFoundException)}
_BY_STATUS[12] = InvalidOperationException  # misuse (the device failure is status 8)


def _check(status: int) -> None:
    if status:
        message = _ffi.lib().satori_hip_last_error().decode("utf-8", "replace")
        raise _BY_STATUS.get(status, SatoriError)(message)


def _ptr(a: np.ndarray) -> ctypes.c_void_p:
    return ctypes.c_void_p(a.ctypes.data)


def _as_u8(data) -> np.ndarray:
    if isinstance(data, (bytes, bytearray, memoryview)):
        return np.frombuffer(bytes(data), dtype=np.uint8)
    return np.ascontiguousarray(data, dtype=np.uint8).reshape(-1)


def _as_f32(a) -> np.ndarray:
    arr = np.asarray(a)
    if arr.dtype != np.float32 or not arr.flags.c_contiguous:
        raise ArgumentException("Vectors must be contiguous float32 arrays.")
    return arr


# ---- shapes ----

class BlockQuantization(enum.IntEnum):
    """src/Satori.Core/BlockQuantization.cs:3."""
    Q8_0 = 0
    Q4_0 = 1
    Q4_K = 2
    Q6_K = 3


_GEOMETRY = {BlockQuantization.Q8_0: (32, 34), BlockQuantization.Q4_0: (32, 18),
             BlockQuantization.Q4_K: (256, 144), BlockQuantization.Q6_K: (256, 210)}


def payload_length(fmt: int, rows: int, columns: int, block_size: int = 0) -> int:
    """Ternary2Shape / QuantizedMatrixShape byte length, with the constructors' checks."""
    out = ctypes.c_int64()
    _check(_ffi.lib().satori_hip_payload_length(int(fmt), rows, columns, block_size, ctypes.byref(out)))
    return out.value


class QuantizedMatrixShape:
    """src/Satori.Core/QuantizedMatrixShape.cs:5-33."""

    def __init__(self, rows: int, columns: int, fmt: BlockQuantization):
        self.format = BlockQuantization(fmt) if int(fmt) in _GEOMETRY else fmt
        self.byte_length = payload_length(int(fmt), rows, columns)
        self.rows, self.columns = rows, columns
        self.block_elements, self.block_bytes = _GEOMETRY[self.format]

    def __eq__(self, other):
        return isinstance(other, QuantizedMatrixShape) and (self.rows, self.columns, self.format) == (
            other.rows, other.columns, other.format)

    def __repr__(self):
        return f"QuantizedMatrixShape({self.rows}, {self.columns}, {self.format.name})"


def quantize_weights(weights, rows: int, columns: int, fmt: BlockQuantization) -> np.ndarray:
    """Round-to-nearest Q8_0/Q4_0/Q4_K/Q6_K payload for synthetic matrices (no reference counterpart)."""
    w = np.ascontiguousarray(weights, dtype=np.float32).reshape(-1)
    if w.size != rows * columns:
        raise ArgumentException("Weights must match matrix dimensions.")
    out = np.zeros(payload_length(int(fmt), rows, columns), dtype=np.uint8)
    _check(_ffi.lib().satori_hip_quantize_weights(int(fmt), _ptr(w), rows, columns, _ptr(out), out.size))
    return out


# ---- device ----

def device_count() -> int:
    n = ctypes.c_int()
    _check(_ffi.lib().satori_hip_device_count(ctypes.byref(n)))
    return n.value


class HipContext:
    """One gfx950 device, one stream: the IQuantizedMatrixFactory of this backend
    (stands where VulkanContext does, src/Satori.Backends.Vulkan/VulkanContext.cs:11)."""

    def __init__(self, device: int = 0):
        handle = ctypes.c_void_p()
        _check(_ffi.lib().satori_hip_context_create(device, ctypes.byref(handle)))
        self._handle = handle
        self.device = device

    @property
    def handle(self) -> ctypes.c_void_p:
        return self._handle

    @property
    def stream(self) -> int:
        s = ctypes.c_void_p()
        _check(_ffi.lib().satori_hip_context_stream(self._handle, ctypes.byref(s)))
        return s.value or 0

    def create(self, payload, shape: QuantizedMatrixShape) -> "HipQuantizedMatrix":
        """IQuantizedMatrixFactory.Create: validates, copies to the device, returns executable weights."""
        data = _as_u8(payload)
        handle = ctypes.c_void_p()
        _check(_ffi.lib().satori_hip_quantized_create(self._handle, shape.rows, shape.columns, int(shape.format),
                                                      _ptr(data), data.size, ctypes.byref(handle)))
        return HipQuantizedMatrix(self, handle)

    def create_ternary2(self, rows: int, columns: int, block_size: int, payload) -> "HipQuantizedMatrix":
        data = _as_u8(payload)
        handle = ctypes.c_void_p()
        _check(_ffi.lib().satori_hip_ternary2_create(self._handle, rows, columns, block_size, _ptr(data), data.size,
                                                     ctypes.byref(handle)))
        return HipQuantizedMatrix(self, handle)

    def open_ternary2(self, path: str) -> "HipQuantizedMatrix":
        handle = ctypes.c_void_p()
        _check(_ffi.lib().satori_hip_ternary2_open(self._handle, str(path).encode(), ctypes.byref(handle)))
        return HipQuantizedMatrix(self, handle)

    def create_bitplane(self, rows: int, columns: int, block_size: int, payload) -> "HipQuantizedMatrix":
        data = _as_u8(payload)
        handle = ctypes.c_void_p()
        _check(_ffi.lib().satori_hip_bitplane_create(self._handle, rows, columns, block_size, _ptr(data), data.size,
                                                     ctypes.byref(handle)))
        return HipQuantizedMatrix(self, handle)

    def open_bitplane(self, path: str) -> "HipQuantizedMatrix":
        handle = ctypes.c_void_p()
        _check(_ffi.lib().satori_hip_bitplane_open(self._handle, str(path).encode(), ctypes.byref(handle)))
        return HipQuantizedMatrix(self, handle)

    def capture_begin(self) -> None:
        """Starts recording the work enqueued on the context stream (satori_hip_capture_begin)."""
        _check(_ffi.lib().satori_hip_capture_begin(self._handle))

    def capture_end(self) -> "HipStep":
        """Ends the recording; the recorded work becomes a replayable step (satori_hip_capture_end)."""
        handle = ctypes.c_void_p()
        _check(_ffi.lib().satori_hip_capture_end(self._handle, ctypes.byref(handle)))
        return HipStep(self, handle=handle)

    def quantize_q8k(self, x) -> np.ndarray:
        """Q8KCodec.QuantizeRow on the device (src/Satori.Core/Q8KCodec.cs:85-93)."""
        xv = _as_f32(x).reshape(-1)
        out = np.zeros((xv.size // 256) * 292 if xv.size % 256 == 0 else 0, dtype=np.uint8)
        _check(_ffi.lib().satori_hip_quantize_q8k(self._handle, _ptr(xv), xv.size, _ptr(out), out.size))
        return out

    # Device buffers (for the *_device entry points and groups).
    def alloc(self, nbytes: int) -> int:
        p = ctypes.c_void_p()
        _check(_ffi.lib().satori_hip_device_alloc(self._handle, nbytes, ctypes.byref(p)))
        return p.value

    def free(self, device_ptr: int) -> None:
        _check(_ffi.lib().satori_hip_device_free(self._handle, ctypes.c_void_p(device_ptr)))

    def upload(self, device_ptr: int, array: np.ndarray) -> None:
        a = np.ascontiguousarray(array)
        _check(_ffi.lib().satori_hip_copy(self._handle, ctypes.c_void_p(device_ptr), _ptr(a), a.nbytes, 1))

    def download(self, array: np.ndarray, device_ptr: int) -> np.ndarray:
        if not array.flags.c_contiguous:
            raise ArgumentException("Destination must be contiguous.")
        _check(_ffi.lib().satori_hip_copy(self._handle, _ptr(array), ctypes.c_void_p(device_ptr), array.nbytes, 2))
        return array

    def copy_device(self, destination_ptr: int, source_ptr: int, nbytes: int) -> None:
        _check(_ffi.lib().satori_hip_copy(self._handle, ctypes.c_void_p(destination_ptr), ctypes.c_void_p(source_ptr),
                                          nbytes, 3))

    def synchronize(self) -> None:
        _check(_ffi.lib().satori_hip_synchronize(self._handle))

    def dispose(self) -> None:
        if self._handle:
            _check(_ffi.lib().satori_hip_context_destroy(self._handle))

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.dispose()


class HipQuantizedMatrix:
    """Resident immutable weights (IQuantizedMatrix, src/Satori.Core/IQuantizedMatrix.cs:4-8)."""

    def __init__(self, context: HipContext, handle: ctypes.c_void_p):
        self.context = context
        self._handle = handle
        r, c, f, b = ctypes.c_int(), ctypes.c_int(), ctypes.c_int(), ctypes.c_int()
        n = ctypes.c_int64()
        _check(_ffi.lib().satori_hip_matrix_shape(handle, ctypes.byref(r), ctypes.byref(c), ctypes.byref(f),
                                                  ctypes.byref(b), ctypes.byref(n)))
        self.rows, self.columns, self.format, self.block_size, self.byte_length = (
            r.value, c.value, f.value, b.value, n.value)

    @property
    def handle(self) -> ctypes.c_void_p:
        return self._handle

    def execute(self, input, output) -> None:
        """Synchronous MatVec; output is written only on success."""
        x, y = _as_f32(input), _as_f32(output)
        _check(_ffi.lib().satori_hip_matvec(self._handle, _ptr(x), x.size, _ptr(y), y.size))

    def execute_batch(self, input, positions: int, output) -> None:
        """QuantizedMatVec.ExecuteBatch semantics: [positions][C] -> [positions][R]."""
        x, y = _as_f32(input), _as_f32(output)
        _check(_ffi.lib().satori_hip_matvec_batch(self._handle, _ptr(x), x.size, positions, _ptr(y), y.size))

    def execute_device(self, input_ptr: int, output_ptr: int, stream: int = 0) -> None:
        _check(_ffi.lib().satori_hip_matvec_device(self._handle, ctypes.c_void_p(input_ptr),
                                                   ctypes.c_void_p(output_ptr), ctypes.c_void_p(stream)))

    def execute_batch_device(self, input_ptr: int, positions: int, output_ptr: int, stream: int = 0) -> None:
        _check(_ffi.lib().satori_hip_matvec_batch_device(self._handle, ctypes.c_void_p(input_ptr), positions,
                                                         ctypes.c_void_p(output_ptr), ctypes.c_void_p(stream)))

    def decode_row_device(self, row: int, output_ptr: int, stream: int = 0) -> None:
        """GgufQuantizedMatrix.ReadRow on the device: row `row` decoded to FP32 at output_ptr (columns floats)."""
        _check(_ffi.lib().satori_hip_matrix_decode_row(self._handle, row, ctypes.c_void_p(output_ptr),
                                                       ctypes.c_void_p(stream)))

    def read_row(self, row: int, output) -> None:
        """GgufQuantizedMatrix.ReadRow (src/Satori.Formats.Gguf/GgufQuantizedMatrix.cs:54-61)."""
        out = _as_f32(output)
        if out.size != self.columns:
            raise ArgumentOutOfRangeException("Specified argument was out of the range of valid values. (Parameter 'row')")
        with _DeviceArrays(self.context, out) as (dy,):
            self.decode_row_device(row, dy)
            self.context.download(out, dy)

    def clone(self) -> "HipQuantizedMatrix":
        handle = ctypes.c_void_p()
        _check(_ffi.lib().satori_hip_matrix_clone(self._handle, ctypes.byref(handle)))
        return HipQuantizedMatrix(self.context, handle)

    def dispose(self) -> None:
        _check(_ffi.lib().satori_hip_matrix_destroy(self._handle))

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.dispose()


class HipGroup:
    """One launch over several matrices of one format and width (device input/output pointers)."""

    def __init__(self, context: HipContext, matrices, inputs, outputs, quantized_activations: bool = False):
        n = len(matrices)
        mats = (ctypes.c_void_p * n)(*[m.handle.value for m in matrices])
        ins = (ctypes.c_void_p * n)(*inputs)
        outs = (ctypes.c_void_p * n)(*outputs)
        handle = ctypes.c_void_p()
        _check(_ffi.lib().satori_hip_group_create(context.handle, mats, n, ins, outs, int(quantized_activations),
                                                  ctypes.byref(handle)))
        self._handle = handle

    def execute(self, stream: int = 0) -> None:
        _check(_ffi.lib().satori_hip_group_execute(self._handle, ctypes.c_void_p(stream)))

    def execute_batch(self, positions: int, stream: int = 0) -> None:
        """Every member over `positions` positions (inputs [positions][columns], outputs [positions][rows]),
        as ExecuteBatch per member; K-format groups with quantized activations only. Members that share an
        input share its Q8_K quantization (the prefill's q/k/v and gate/up, DenseForward.LayerBatch)."""
        _check(_ffi.lib().satori_hip_group_execute_batch(self._handle, int(positions), ctypes.c_void_p(stream)))

    def set_input_add_rms_norm(self, residual: int, addend: int, weights: int, epsilon: float,
                               residual_out: int = 0) -> None:
        """The group's input becomes RmsNorm(residual + addend, weights, epsilon) computed inside its launch
        (addend 0: RmsNorm(residual)); residual + addend is also written to residual_out when given. Device
        pointers; bit-identical to the separate add / RmsNorm operators."""
        _check(_ffi.lib().satori_hip_group_set_input(self._handle, 1, ctypes.c_void_p(residual),
                                                     ctypes.c_void_p(addend or None), ctypes.c_void_p(weights),
                                                     float(epsilon), ctypes.c_void_p(residual_out or None)))

    def set_input_swiglu(self, gate: int, up: int) -> None:
        """The group's input becomes SwiGlu(gate, up) computed inside its launch (device pointers)."""
        _check(_ffi.lib().satori_hip_group_set_input(self._handle, 2, ctypes.c_void_p(gate), ctypes.c_void_p(up),
                                                     None, 0.0, None))

    def set_input_q8k(self, q8k: int) -> None:
        """The group reads its input already quantized to Q8_K at `q8k` (device bytes written by its producer,
        DeviceOps.swiglu_q8k / quantize_q8k) instead of quantizing it."""
        _check(_ffi.lib().satori_hip_group_set_input(self._handle, 3, ctypes.c_void_p(q8k), None, None, 0.0, None))

    def set_input_plain(self) -> None:
        """The group reads its creation inputs again."""
        _check(_ffi.lib().satori_hip_group_set_input(self._handle, 0, None, None, None, 0.0, None))

    def set_output_swiglu(self, activated: int, q8k: int = 0) -> None:
        """A two-member group (gate, up; equal row counts, a multiple of 256) also writes SwiGlu(gate, up) to
        `activated` inside its launch (device pointer), bit-identical to DeviceOps.swiglu over the two outputs;
        with `q8k`, also that vector's Q8_K bytes, as DeviceOps.swiglu_q8k writes them (a down group reads
        them through set_input_q8k)."""
        _check(_ffi.lib().satori_hip_group_set_output(self._handle, 1, ctypes.c_void_p(activated),
                                                      ctypes.c_void_p(q8k or None)))

    def set_output_plain(self) -> None:
        """The group writes its members' outputs only."""
        _check(_ffi.lib().satori_hip_group_set_output(self._handle, 0, None, None))

    def dispose(self) -> None:
        _check(_ffi.lib().satori_hip_group_destroy(self._handle))


class HipStep:
    """An ordered list of groups captured once and replayed as one HIP graph (the projection sequence of a
    decode step). The groups must stay alive while the step exists."""

    def __init__(self, context: HipContext, groups=None, handle: ctypes.c_void_p | None = None):
        if handle is None:
            n = len(groups)
            handles = (ctypes.c_void_p * n)(*[g._handle.value for g in groups])
            handle = ctypes.c_void_p()
            _check(_ffi.lib().satori_hip_step_create(context.handle, handles, n, ctypes.byref(handle)))
        self._handle = handle

    def execute(self, stream: int = 0) -> None:
        _check(_ffi.lib().satori_hip_step_execute(self._handle, ctypes.c_void_p(stream)))

    def dispose(self) -> None:
        _check(_ffi.lib().satori_hip_step_destroy(self._handle))


_default_lock = threading.Lock()
_default: HipContext | None = None


def default_context() -> HipContext:
    """Process-wide context on device 0, created on first use (the static surfaces use it)."""
    global _default
    with _default_lock:
        if _default is None:
            _default = HipContext(0)
        return _default


# ---- Ternary2 ----

class Ternary2Matrix:
    """Owned, validated Ternary2 weights (src/Satori.Core/Ternary2Matrix.cs:6-124). The device copy is made
    on first execution and kept with the matrix."""

    def __init__(self, rows: int, columns: int, block_size: int, data: np.ndarray):
        self.rows, self.columns, self.block_size = rows, columns, block_size
        self._data = data
        self._device: HipQuantizedMatrix | None = None

    @property
    def byte_length(self) -> int:
        return self._data.size

    @property
    def data(self) -> np.ndarray:
        return self._data

    @staticmethod
    def quantize(weights, rows: int, columns: int, block_size: int = 64) -> "Ternary2Matrix":
        """Ternary2Matrix.Quantize (Ternary2Matrix.cs:38-71)."""
        length = payload_length(TERNARY2, rows, columns, block_size)
        w = np.ascontiguousarray(weights, dtype=np.float32).reshape(-1)
        if w.size != rows * columns:
            raise ArgumentException("Weights must match matrix dimensions.")
        out = np.zeros(length, dtype=np.uint8)
        _check(_ffi.lib().satori_hip_ternary2_quantize(_ptr(w), rows, columns, block_size, _ptr(out), out.size))
        return Ternary2Matrix(rows, columns, block_size, out)

    @staticmethod
    def from_packed(rows: int, columns: int, block_size: int, data) -> "Ternary2Matrix":
        """Ternary2Matrix.FromPacked (Ternary2Matrix.cs:73-81): copies and validates."""
        owned = _as_u8(data).copy()
        _check(_ffi.lib().satori_hip_ternary2_validate(rows, columns, block_size, _ptr(owned), owned.size))
        return Ternary2Matrix(rows, columns, block_size, owned)

    def copy_data_to(self, destination: np.ndarray) -> None:
        destination[: self._data.size] = self._data

    def save(self, path: str) -> None:
        """Ternary2Matrix.Save (Ternary2Matrix.cs:29-36): STQ2 header + payload, new file only."""
        header = bytearray(32)
        header[0:4] = b"STQ2"
        header[4:6] = (1).to_bytes(2, "little")
        header[6:8] = (32).to_bytes(2, "little")
        header[8:12] = self.rows.to_bytes(4, "little", signed=True)
        header[12:16] = self.columns.to_bytes(4, "little", signed=True)
        header[16:20] = self.block_size.to_bytes(4, "little", signed=True)
        header[24:32] = self.byte_length.to_bytes(8, "little", signed=True)
        with open(path, "xb") as f:
            f.write(bytes(header))
            f.write(self._data.tobytes())

    def device(self, context: HipContext | None = None) -> HipQuantizedMatrix:
        if self._device is None:
            ctx = context or default_context()
            self._device = ctx.create_ternary2(self.rows, self.columns, self.block_size, self._data)
        return self._device


class Ternary2MatVec:
    """src/Satori.Core/Ternary2MatVec.cs:7-77 with the HIP backend."""

    @staticmethod
    def execute(matrix: Ternary2Matrix, input, output, context: HipContext | None = None) -> None:
        if matrix is None:
            raise ArgumentNullException("Value cannot be null. (Parameter 'matrix')")
        matrix.device(context).execute(input, output)


class TernaryBitplaneMatrix:
    """src/Satori.Core/TernaryBitplaneMatrix.cs:6-118: ternary weights as separate positive and negative
    bitplanes (same shape and byte length as Ternary2). Conversions and validation run in the library; the
    device copy (made on first execution) is the lossless Ternary2 equivalent."""

    def __init__(self, rows: int, columns: int, block_size: int, data: np.ndarray):
        self.rows, self.columns, self.block_size = rows, columns, block_size
        self._data = data
        self._device: HipQuantizedMatrix | None = None

    @property
    def byte_length(self) -> int:
        return self._data.size

    @property
    def data(self) -> np.ndarray:
        return self._data

    def copy_data_to(self, destination: np.ndarray) -> None:
        destination[: self._data.size] = self._data

    @staticmethod
    def from_ternary2(matrix: Ternary2Matrix) -> "TernaryBitplaneMatrix":
        """FromTernary2 (TernaryBitplaneMatrix.cs:19-36)."""
        out = np.zeros(matrix.byte_length, dtype=np.uint8)
        _check(_ffi.lib().satori_hip_bitplane_from_ternary2(matrix.rows, matrix.columns, matrix.block_size,
                                                            _ptr(matrix.data), matrix.byte_length, _ptr(out), out.size))
        return TernaryBitplaneMatrix(matrix.rows, matrix.columns, matrix.block_size, out)

    def to_ternary2(self) -> Ternary2Matrix:
        """ToTernary2 (TernaryBitplaneMatrix.cs:38-54)."""
        out = np.zeros(self.byte_length, dtype=np.uint8)
        _check(_ffi.lib().satori_hip_bitplane_to_ternary2(self.rows, self.columns, self.block_size, _ptr(self._data),
                                                          self.byte_length, _ptr(out), out.size))
        return Ternary2Matrix.from_packed(self.rows, self.columns, self.block_size, out)

    @staticmethod
    def from_packed(rows: int, columns: int, block_size: int, payload) -> "TernaryBitplaneMatrix":
        """FromPacked (TernaryBitplaneMatrix.cs:56-62): copies and validates."""
        owned = _as_u8(payload).copy()
        _check(_ffi.lib().satori_hip_bitplane_validate(rows, columns, block_size, _ptr(owned), owned.size))
        return TernaryBitplaneMatrix(rows, columns, block_size, owned)

    def save(self, path: str) -> None:
        """Save (TernaryBitplaneMatrix.cs:87-96): the STQ2 header with magic "STB1", then the payload."""
        header = bytearray(32)
        header[0:4] = b"STB1"
        header[4:6] = (1).to_bytes(2, "little")
        header[6:8] = (32).to_bytes(2, "little")
        header[8:12] = self.rows.to_bytes(4, "little", signed=True)
        header[12:16] = self.columns.to_bytes(4, "little", signed=True)
        header[16:20] = self.block_size.to_bytes(4, "little", signed=True)
        header[24:32] = self.byte_length.to_bytes(8, "little", signed=True)
        with open(path, "xb") as f:
            f.write(bytes(header))
            f.write(self._data.tobytes())

    @staticmethod
    def load(path: str) -> "TernaryBitplaneMatrix":
        """Load (TernaryBitplaneMatrix.cs:98-117): every file defect raises InvalidDataException."""
        rows, columns, block, length = ctypes.c_int(), ctypes.c_int(), ctypes.c_int(), ctypes.c_int64()
        p = os.fsencode(path)
        _check(_ffi.lib().satori_hip_bitplane_load(p, ctypes.byref(rows), ctypes.byref(columns), ctypes.byref(block),
                                                   None, 0, ctypes.byref(length)))
        out = np.zeros(length.value, dtype=np.uint8)
        _check(_ffi.lib().satori_hip_bitplane_load(p, None, None, None, _ptr(out), out.size, ctypes.byref(length)))
        return TernaryBitplaneMatrix(rows.value, columns.value, block.value, out)

    def device(self, context: HipContext | None = None) -> HipQuantizedMatrix:
        if self._device is None:
            ctx = context or default_context()
            self._device = ctx.create_bitplane(self.rows, self.columns, self.block_size, self._data)
        return self._device


class TernaryBitplaneMatVec:
    """src/Satori.Core/TernaryBitplaneMatVec.cs:6-54 with the HIP backend."""

    @staticmethod
    def execute(matrix: TernaryBitplaneMatrix, input, output, context: HipContext | None = None) -> None:
        if matrix is None:
            raise ArgumentNullException("Value cannot be null. (Parameter 'matrix')")
        matrix.device(context).execute(input, output)


class MappedTernary2Matrix:
    """src/Satori.Core/MappedTernary2Matrix.cs:4-56: opens and validates an STQ2 file once, then executes
    on its resident device copy."""

    def __init__(self, path: str, context: HipContext | None = None):
        self._matrix = (context or default_context()).open_ternary2(path)
        self.rows, self.columns = self._matrix.rows, self._matrix.columns
        self.block_size, self.byte_length = self._matrix.block_size, self._matrix.byte_length

    def execute(self, input, output) -> None:
        self._matrix.execute(input, output)

    def dispose(self) -> None:
        self._matrix.dispose()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.dispose()


# ---- GGUF block formats ----

class QuantizedMatVec:
    """src/Satori.Core/QuantizedMatVec.cs:9-370 with the HIP backend. The static calls upload the payload per
    call, as the reference reads it per call; resident use goes through HipContext.create."""

    @staticmethod
    def validate_payload(data, shape: QuantizedMatrixShape) -> None:
        d = _as_u8(data)
        _check(_ffi.lib().satori_hip_quantized_validate(shape.rows, shape.columns, int(shape.format), _ptr(d), d.size))

    @staticmethod
    def execute(data, shape: QuantizedMatrixShape, input, output, context: HipContext | None = None) -> None:
        with (context or default_context()).create(data, shape) as m:
            m.execute(input, output)

    @staticmethod
    def execute_batch(data, shape: QuantizedMatrixShape, input, positions: int, output, threads: int = 1,
                      context: HipContext | None = None) -> None:
        if threads <= 0:
            raise ArgumentOutOfRangeException("threads must be positive.")
        with (context or default_context()).create(data, shape) as m:
            m.execute_batch(input, positions, output)


class Q8KCodec:
    """src/Satori.Core/Q8KCodec.cs: the activation codec, quantized on the device."""
    ELEMENTS_PER_BLOCK = 256
    BYTES_PER_BLOCK = 292

    @staticmethod
    def quantize_row(input, context: HipContext | None = None) -> np.ndarray:
        return (context or default_context()).quantize_q8k(input)


# ---- GGUF containers (src/Satori.Formats.Gguf) ----

class GgufTensor:
    """src/Satori.Formats.Gguf/GgufTensor.cs:5-20: name, dimensions (dims[0] contiguous), type id, absolute
    payload offset, payload byte length."""

    __slots__ = ("name", "dimensions", "type", "offset", "byte_length")

    def __init__(self, name, dimensions, type_, offset, byte_length):
        self.name, self.dimensions, self.type = name, tuple(dimensions), type_
        self.offset, self.byte_length = offset, byte_length

    def __repr__(self) -> str:
        return (f"GgufTensor({self.name!r}, dims={self.dimensions}, type={self.type}, offset={self.offset}, "
                f"length={self.byte_length})")


class GgufMetadata:
    """src/Satori.Formats.Gguf/GgufMetadata.cs:3-4; element_type / element_count are None for scalars."""

    __slots__ = ("key", "type", "offset", "byte_length", "element_type", "element_count")

    def __init__(self, key, type_, offset, byte_length, element_type, element_count):
        self.key, self.type, self.offset, self.byte_length = key, type_, offset, byte_length
        self.element_type = None if element_type < 0 else element_type
        self.element_count = None if element_count < 0 else element_count


class GgufFile:
    """src/Satori.Formats.Gguf/GgufFile.cs:10-207: a GGUF v3 file mapped read-only with its catalogue parsed
    strictly by the library (limits and failure kinds of GgufFile.Parse); windows are read from the mapping."""

    def __init__(self, path: str):
        handle = ctypes.c_void_p()
        _check(_ffi.lib().satori_hip_gguf_open(os.fsencode(path), ctypes.byref(handle)))
        self._handle = handle
        lib = _ffi.lib()
        offset = ctypes.c_int64()
        _check(lib.satori_hip_gguf_data_offset(handle, ctypes.byref(offset)))
        self.data_offset = offset.value
        count = ctypes.c_int64()
        _check(lib.satori_hip_gguf_tensor_count(handle, ctypes.byref(count)))
        self._index = {}
        self.tensors = {}
        for i in range(count.value):
            name, rank, dims = ctypes.c_char_p(), ctypes.c_int(), (ctypes.c_int64 * 4)()
            type_, off, length = ctypes.c_uint32(), ctypes.c_int64(), ctypes.c_int64()
            _check(lib.satori_hip_gguf_tensor_info(handle, i, ctypes.byref(name), ctypes.byref(rank), dims,
                                                   ctypes.byref(type_), ctypes.byref(off), ctypes.byref(length)))
            key = name.value.decode("utf-8")
            self._index[key] = i
            self.tensors[key] = GgufTensor(key, dims[:rank.value], type_.value, off.value, length.value)
        _check(lib.satori_hip_gguf_metadata_count(handle, ctypes.byref(count)))
        self._meta_index = {}
        self.metadata = {}
        for i in range(count.value):
            key, type_, off, length = ctypes.c_char_p(), ctypes.c_uint32(), ctypes.c_int64(), ctypes.c_int64()
            et, ec = ctypes.c_int64(), ctypes.c_int64()
            _check(lib.satori_hip_gguf_metadata_info(handle, i, ctypes.byref(key), ctypes.byref(type_),
                                                     ctypes.byref(off), ctypes.byref(length), ctypes.byref(et),
                                                     ctypes.byref(ec)))
            k = key.value.decode("utf-8")
            self._meta_index[k] = i
            self.metadata[k] = GgufMetadata(k, type_.value, off.value, length.value, et.value, ec.value)

    @property
    def handle(self) -> ctypes.c_void_p:
        return self._handle

    def tensor_index(self, name: str) -> int:
        index = ctypes.c_int64()
        _check(_ffi.lib().satori_hip_gguf_tensor_find(self._handle, name.encode("utf-8"), ctypes.byref(index)))
        return index.value

    def read_tensor(self, name: str, offset: int, length: int) -> bytes:
        """GgufFile.ReadTensor (GgufFile.cs:42-49): a copy of the window [offset, offset + length)."""
        index = self.tensor_index(name)
        p = ctypes.c_void_p()
        _check(_ffi.lib().satori_hip_gguf_tensor_window(self._handle, index, offset, length, ctypes.byref(p)))
        return ctypes.string_at(p.value, length) if length else b""

    def read_metadata(self, key: str) -> bytes:
        """GgufFile.ReadMetadata (GgufFile.cs:51-56): the value bytes as stored."""
        index = ctypes.c_int64()
        _check(_ffi.lib().satori_hip_gguf_metadata_find(self._handle, key.encode("utf-8"), ctypes.byref(index)))
        p, n = ctypes.c_void_p(), ctypes.c_int64()
        _check(_ffi.lib().satori_hip_gguf_metadata_window(self._handle, index.value, ctypes.byref(p), ctypes.byref(n)))
        return ctypes.string_at(p.value, n.value) if n.value else b""

    _SCALARS = {0: "<B", 1: "<b", 2: "<H", 3: "<h", 4: "<I", 5: "<i", 6: "<f", 10: "<Q", 11: "<q", 12: "<d"}

    def read_scalar(self, key: str):
        """GgufFile.ReadScalar (GgufFile.cs:58-76)."""
        import struct
        entry = self.metadata.get(key)
        if entry is None:
            self.read_metadata(key)  # raises KeyNotFoundException
        if entry.type == 9:
            raise InvalidOperationException("Use scoped access for arrays.")
        raw = self.read_metadata(key)
        if entry.type == 7:
            return raw[0] != 0
        if entry.type == 8:
            return raw[8:].decode("utf-8")
        return struct.unpack(self._SCALARS[entry.type], raw)[0]

    def dispose(self) -> None:
        _check(_ffi.lib().satori_hip_gguf_close(self._handle))

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.dispose()


_GGUF_FORMATS = {8: 0, 2: 1, 12: 2, 14: 3}  # GGUF type id -> BlockQuantization (GgufQuantizedMatrix.cs:20-26)


class GgufQuantizedMatrix:
    """src/Satori.Formats.Gguf/GgufQuantizedMatrix.cs:6-86: a rank-2 Q8_0/Q4_0/Q4_K/Q6_K tensor of a GgufFile.
    The constructor applies the reference's checks (type, rank, Int32 limits, payload validation);
    create_execution uploads it to a resident device matrix (block scales checked again on the device)."""

    def __init__(self, file: GgufFile, name: str):
        tensor = file.tensors[name] if name in file.tensors else None
        if tensor is None:
            file.tensor_index(name)  # raises KeyNotFoundException
        dims = tensor.dimensions
        if (tensor.type not in _GGUF_FORMATS or len(dims) != 2 or tensor.byte_length > 0x7FFFFFFF
                or any(d > 0x7FFFFFFF for d in dims)):
            raise NotSupportedException("MatVec requires a rank-2 Q8_0/Q4_0/Q4_K/Q6_K tensor within Int32 limits.")
        self.shape = QuantizedMatrixShape(dims[1], dims[0], BlockQuantization(_GGUF_FORMATS[tensor.type]))
        self.name = name
        self._file = file
        self._resident = None
        QuantizedMatVec.validate_payload(file.read_tensor(name, 0, self.shape.byte_length), self.shape)

    def create_execution(self, context: "HipContext | None" = None) -> "HipQuantizedMatrix":
        """CreateExecution(factory) (GgufQuantizedMatrix.cs:31-36): a device copy owned by the caller."""
        ctx = context or default_context()
        handle = ctypes.c_void_p()
        _check(_ffi.lib().satori_hip_gguf_matrix_create(ctx.handle, self._file.handle, self._file.tensor_index(self.name),
                                                        ctypes.byref(handle)))
        return HipQuantizedMatrix(ctx, handle)

    def _device(self) -> "HipQuantizedMatrix":
        if self._resident is None:
            self._resident = self.create_execution()
        return self._resident

    def execute(self, input, output) -> None:
        self._device().execute(input, output)

    def execute_batch(self, input, positions: int, output, threads: int = 1) -> None:
        if threads <= 0:
            raise ArgumentOutOfRangeException("threads must be positive.")
        self._device().execute_batch(input, positions, output)

    def dispose(self) -> None:
        if self._resident is not None:
            self._resident.dispose()
            self._resident = None


class GgufWeightStore:
    """src/Satori.Formats.Gguf/GgufWeightStore.cs:19-55, projection part: tensors of a GgufFile as resident
    device matrices, created once per name on first use. The store borrows the file."""

    def __init__(self, file: GgufFile, context: "HipContext | None" = None):
        if file is None:
            raise ArgumentNullException("Value cannot be null. (Parameter 'file')")
        self._file = file
        self._context = context
        self._matrices = {}
        self._lock = threading.Lock()

    def has(self, name: str) -> bool:
        return name in self._file.tensors

    def matrix(self, name: str) -> "HipQuantizedMatrix":
        with self._lock:
            m = self._matrices.get(name)
            if m is None:
                m = GgufQuantizedMatrix(self._file, name).create_execution(self._context)
                self._matrices[name] = m
            return m

    def project(self, name: str, input, output) -> None:
        self.matrix(name).execute(input, output)

    def project_batch(self, name: str, input, positions: int, output, threads: int = 1) -> None:
        if threads <= 0:
            raise ArgumentOutOfRangeException("threads must be positive.")
        self.matrix(name).execute_batch(input, positions, output)

    def dispose(self) -> None:
        with self._lock:
            for m in self._matrices.values():
                m.dispose()
            self._matrices.clear()


# ---- decode-step operators (src/Satori.Core/TransformerOps.cs) ----

class _DeviceArrays:
    """Device copies of host float arrays for one operator call (freed on exit)."""

    def __init__(self, context: "HipContext", *arrays):
        self.context, self.arrays, self.ptrs = context, arrays, []

    def __enter__(self):
        for a in self.arrays:
            p = self.context.alloc(max(a.nbytes, 4))
            self.ptrs.append(p)
            if a.nbytes:
                self.context.upload(p, a)
        return self.ptrs

    def __exit__(self, *exc):
        self.context.synchronize()
        for p in self.ptrs:
            self.context.free(p)


class TransformerOps:
    """src/Satori.Core/TransformerOps.cs:5-180 on the device, over host float32 arrays (each call copies in,
    runs on the context stream and copies out). The *_device entry points of the library take device pointers
    for resident pipelines."""

    @staticmethod
    def _ctx(context):
        return context or default_context()

    @staticmethod
    def rms_norm(input, weights, epsilon: float, output, context: "HipContext | None" = None) -> None:
        ctx = TransformerOps._ctx(context)
        x, w, y = _as_f32(input).reshape(-1), _as_f32(weights).reshape(-1), _as_f32(output).reshape(-1)
        if x.size != y.size or w.size != y.size:
            raise ArgumentException("Lengths differ.")
        with _DeviceArrays(ctx, x, w) as (dx, dw):
            _check(_ffi.lib().satori_hip_rms_norm(ctx.handle, ctypes.c_void_p(dx), ctypes.c_void_p(dw), float(epsilon),
                                                  x.size, 1, ctypes.c_void_p(dx), None))
            ctx.download(y, dx)

    @staticmethod
    def rms_norm_heads(vector, weights, epsilon: float, head_dimension: int, context: "HipContext | None" = None) -> None:
        ctx = TransformerOps._ctx(context)
        v, w = _as_f32(vector).reshape(-1), _as_f32(weights).reshape(-1)
        if w.size != head_dimension and head_dimension > 0 and v.size % head_dimension == 0:
            raise ArgumentException("Per-head weights must match the head dimension.")
        with _DeviceArrays(ctx, v, w) as (dv, dw):
            _check(_ffi.lib().satori_hip_rms_norm_heads(ctx.handle, ctypes.c_void_p(dv), ctypes.c_void_p(dw),
                                                        float(epsilon), head_dimension, v.size, None))
            ctx.download(v, dv)

    @staticmethod
    def rope(vector, head_dimension: int, position: int, context: "HipContext | None" = None) -> None:
        ctx = TransformerOps._ctx(context)
        v = _as_f32(vector).reshape(-1)
        with _DeviceArrays(ctx, v) as (dv,):
            _check(_ffi.lib().satori_hip_rope(ctx.handle, ctypes.c_void_p(dv), v.size, head_dimension, position, None))
            ctx.download(v, dv)

    @staticmethod
    def rope_half(vector, head_dimension: int, position: int, frequency_base: float, rotary_dimensions: int,
                  context: "HipContext | None" = None) -> None:
        ctx = TransformerOps._ctx(context)
        v = _as_f32(vector).reshape(-1)
        with _DeviceArrays(ctx, v) as (dv,):
            _check(_ffi.lib().satori_hip_rope_half(ctx.handle, ctypes.c_void_p(dv), v.size, head_dimension, position,
                                                   float(frequency_base), rotary_dimensions, None))
            ctx.download(v, dv)

    @staticmethod
    def swiglu(gate, up, output, context: "HipContext | None" = None) -> None:
        ctx = TransformerOps._ctx(context)
        g, u, y = _as_f32(gate).reshape(-1), _as_f32(up).reshape(-1), _as_f32(output).reshape(-1)
        if g.size != y.size or u.size != y.size:
            raise ArgumentException("Lengths differ.")
        with _DeviceArrays(ctx, g, u) as (dg, du):
            _check(_ffi.lib().satori_hip_swiglu(ctx.handle, ctypes.c_void_p(dg), ctypes.c_void_p(du), g.size,
                                                ctypes.c_void_p(dg), None))
            ctx.download(y, dg)

    @staticmethod
    def add(left, right, output, context: "HipContext | None" = None) -> None:
        ctx = TransformerOps._ctx(context)
        a, b, y = _as_f32(left).reshape(-1), _as_f32(right).reshape(-1), _as_f32(output).reshape(-1)
        if a.size != y.size or b.size != y.size:
            raise ArgumentException("Lengths differ.")
        with _DeviceArrays(ctx, a, b) as (da, db):
            _check(_ffi.lib().satori_hip_add(ctx.handle, ctypes.c_void_p(da), ctypes.c_void_p(db), a.size,
                                             ctypes.c_void_p(da), None))
            ctx.download(y, da)

    @staticmethod
    def grouped_attention(query, keys, values, query_heads: int, kv_heads: int, head_dimension: int, token_count: int,
                          output, context: "HipContext | None" = None) -> None:
        ctx = TransformerOps._ctx(context)
        q, k, v, y = (_as_f32(a).reshape(-1) for a in (query, keys, values, output))
        if head_dimension <= 0 or query_heads <= 0 or kv_heads <= 0 or query_heads % kv_heads or token_count <= 0:
            raise ArgumentException("Invalid grouped-attention dimensions.")
        if q.size != query_heads * head_dimension or y.size != q.size:
            raise ArgumentException("Query or output width does not match the head count.")
        if k.size != token_count * kv_heads * head_dimension or v.size != k.size:
            raise ArgumentException("Key/value width does not match the KV head count.")
        with _DeviceArrays(ctx, q, k, v, y) as (dq, dk, dv, dy):
            _check(_ffi.lib().satori_hip_grouped_attention(ctx.handle, ctypes.c_void_p(dq), ctypes.c_void_p(dk),
                                                           ctypes.c_void_p(dv), query_heads, kv_heads, head_dimension,
                                                           token_count, ctypes.c_void_p(dy), None))
            ctx.download(y, dy)

    @staticmethod
    def attention(query, keys, values, head_dimension: int, token_count: int, output,
                  context: "HipContext | None" = None) -> None:
        """Attention (TransformerOps.cs:61-91): equal query and key/value heads."""
        q = _as_f32(query).reshape(-1)
        if head_dimension <= 0 or q.size == 0 or q.size % head_dimension:
            raise ArgumentException("Invalid attention dimensions.")
        heads = q.size // head_dimension
        TransformerOps.grouped_attention(q, keys, values, heads, heads, head_dimension, token_count, output, context)


class DeviceOps:
    """The decode-step operators over device pointers (ints), enqueued on the context stream (so they can be
    captured with HipContext.capture_begin / capture_end). Argument meaning as TransformerOps."""

    def __init__(self, context: "HipContext"):
        self.context = context
        self._h = context.handle

    @staticmethod
    def _p(v: int) -> ctypes.c_void_p:
        return ctypes.c_void_p(v)

    def rms_norm(self, x: int, weights: int, epsilon: float, length: int, y: int, count: int = 1) -> None:
        _check(_ffi.lib().satori_hip_rms_norm(self._h, self._p(x), self._p(weights), float(epsilon), length, count,
                                              self._p(y), None))

    def rms_norm_heads(self, v: int, weights: int, epsilon: float, head_dim: int, length: int) -> None:
        _check(_ffi.lib().satori_hip_rms_norm_heads(self._h, self._p(v), self._p(weights), float(epsilon), head_dim,
                                                    length, None))

    def rope_half(self, v: int, length: int, head_dim: int, position: int, base: float, rotary: int) -> None:
        _check(_ffi.lib().satori_hip_rope_half(self._h, self._p(v), length, head_dim, position, float(base), rotary,
                                               None))

    def swiglu(self, gate: int, up: int, length: int, out: int) -> None:
        _check(_ffi.lib().satori_hip_swiglu(self._h, self._p(gate), self._p(up), length, self._p(out), None))

    def add(self, left: int, right: int, length: int, out: int) -> None:
        _check(_ffi.lib().satori_hip_add(self._h, self._p(left), self._p(right), length, self._p(out), None))

    def swiglu_q8k(self, gate: int, up: int, length: int, out: int, q8k: int) -> None:
        """SwiGlu with the Q8_K bytes of its output (out may be 0: no FP32 output)."""
        _check(_ffi.lib().satori_hip_swiglu_q8k(self._h, self._p(gate), self._p(up), length,
                                                self._p(out) if out else None, self._p(q8k), None))

    def quantize_q8k(self, x: int, columns: int, positions: int, out: int) -> None:
        """Q8KCodec.QuantizeRow of `positions` device rows into device Q8_K bytes."""
        _check(_ffi.lib().satori_hip_quantize_q8k_device(self._h, self._p(x), columns, positions, self._p(out), None))

    def add_rms_norm(self, residual: int, addend: int, weights: int, epsilon: float, length: int, normed: int) -> None:
        _check(_ffi.lib().satori_hip_add_rms_norm(self._h, self._p(residual), self._p(addend), self._p(weights),
                                                  float(epsilon), length, self._p(normed), None))

    def add_rms_norm_q8k(self, residual: int, addend: int, weights: int, epsilon: float, length: int, normed: int,
                         q8k: int) -> None:
        """add_rms_norm with the Q8_K bytes of `normed` written to q8k as well (for a group reading Q8_K)."""
        _check(_ffi.lib().satori_hip_add_rms_norm_q8k(self._h, self._p(residual), self._p(addend), self._p(weights),
                                                      float(epsilon), length, self._p(normed), self._p(q8k), None))

    def attention_inputs(self, q: int, q_bias: int, k: int, k_bias: int, k_out: int, v: int, v_bias: int, v_out: int,
                         heads: int, kv_heads: int, head_dim: int, position: int, base: float, rotary: int) -> None:
        """Biases may be 0 (none)."""
        _check(_ffi.lib().satori_hip_attention_inputs(self._h, self._p(q), self._p(q_bias), self._p(k), self._p(k_bias),
                                                      self._p(k_out), self._p(v), self._p(v_bias), self._p(v_out), heads,
                                                      kv_heads, head_dim, position, float(base), rotary, None))

    def attention_decode(self, q: int, q_bias: int, k: int, k_bias: int, v: int, v_bias: int, keys: int, values: int,
                         heads: int, kv_heads: int, head_dim: int, position: int, base: float, rotary: int,
                         out: int, rope_table: int = 0) -> None:
        """attention_inputs (cache slots of row `position`) then grouped_attention over position + 1 rows, one
        launch fewer; biases and rope_table (a rope_table() table) may be 0."""
        _check(_ffi.lib().satori_hip_attention_decode(self._h, self._p(q), self._p(q_bias), self._p(k), self._p(k_bias),
                                                      self._p(v), self._p(v_bias), self._p(keys), self._p(values), heads,
                                                      kv_heads, head_dim, position, float(base), rotary,
                                                      self._p(rope_table) if rope_table else None, self._p(out), None))

    def rope_table(self, positions: int, rotary: int, base: float, table: int) -> None:
        """RoPE sines and cosines of positions 0 .. positions - 1 into `table` (positions * rotary doubles)."""
        _check(_ffi.lib().satori_hip_rope_table(self._h, positions, rotary, float(base), self._p(table), None))

    def grouped_attention_static(self, q: int, k: int, v: int, query_heads: int, kv_heads: int, head_dim: int,
                                 tokens: int, out: int, stream: int = 0) -> None:
        """grouped_attention with no allocation (satori_hip_grouped_attention_static): the split partials go to
        the device's static 4 MiB workspace, shared by every such call on the device."""
        _check(_ffi.lib().satori_hip_grouped_attention_static(self._h, self._p(q), self._p(k), self._p(v),
                                                              query_heads, kv_heads, head_dim, tokens, self._p(out),
                                                              self._p(stream) if stream else None))

    def grouped_attention(self, q: int, k: int, v: int, query_heads: int, kv_heads: int, head_dim: int, tokens: int,
                          out: int, stream: int = 0) -> None:
        """`stream`: a HIP stream handle (0: the context stream)."""
        _check(_ffi.lib().satori_hip_grouped_attention(self._h, self._p(q), self._p(k), self._p(v), query_heads,
                                                       kv_heads, head_dim, tokens, self._p(out),
                                                       self._p(stream) if stream else None))
