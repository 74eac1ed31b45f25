"""Per-layer host API over libgguf_hip, mirroring the reference's WebGPU engine.

Reference interfaces (webgpu/src/...):
* ``GGUFWeight {data, ggmlType, byteOffset?}``       engine/forward-pass.ts:89-98
* ``dispatchMatmulGGUF(aBuf, gg, cBuf, M, N, K, label, io?)``   forward-pass.ts:1496-1544
* ``dispatchProjection(inputBuf, lw, proj, outputBuf, M, N, K, label, gpuDequant?, io?)``
                                                      forward-pass.ts:1576-1629
* gate+up row concatenation                          forward-pass.ts:740-791
* ``repackGGUFForGPU(ggmlType, data, n)``             model/gguf-dequant.ts:809-840
* ``dequantGGML(ggmlType, data, n)``                  model/gguf-dequant.ts:844-868

Buffers are torch tensors on the current HIP device; kernels are enqueued on
torch's current stream, and nothing here synchronizes with the host.  There is
no CPU path: every quantized operation runs in libgguf_hip and raises if it
cannot.
"""

from __future__ import annotations

import dataclasses
from typing import Optional

import numpy as np
import torch

from . import _native
from .ggml import (F16, F32, GGML_TYPE_NAMES, TILE_ROWS, check_kernel_type, ggml_type_traits,
                   raw_row_bytes, tile_row_bytes, tiled_bytes)

_X_TYPES = {torch.float32: F32, torch.float16: F16}


def _stream(dev: torch.device) -> int:
    return torch.cuda.current_stream(dev).cuda_stream


def _as_device_u8(data, device) -> torch.Tensor:
    if isinstance(data, torch.Tensor):
        t = data
    elif isinstance(data, np.ndarray):
        t = torch.from_numpy(np.ascontiguousarray(data).view(np.uint8).reshape(-1))
    elif isinstance(data, (bytes, bytearray, memoryview)):
        t = torch.frombuffer(bytearray(data), dtype=torch.uint8)
    else:
        raise TypeError(f"unsupported buffer type {type(data).__name__}")
    if t.dtype != torch.uint8:
        t = t.contiguous().view(torch.uint8)
    t = t.reshape(-1)
    if not t.is_cuda:
        t = t.to(device if device is not None else "cuda", non_blocking=False)
    return t.contiguous()


@dataclasses.dataclass
class GGUFWeight:
    """A quantized ``[n, k]`` matrix resident in HBM (forward-pass.ts:89-98).

    ``data`` is a uint8 device tensor holding the weight in the row-tile
    layout (``tiled_bytes(ggml_type, n, k)`` bytes: ``n`` rows rounded up to
    whole 16-row tiles) starting at ``byte_offset``.
    """

    data: torch.Tensor
    ggml_type: int
    n: int
    k: int
    byte_offset: int = 0

    def __post_init__(self):
        check_kernel_type(self.ggml_type)
        if self.data.dtype != torch.uint8 or not self.data.is_cuda:
            raise ValueError("GGUFWeight.data must be a uint8 tensor on a HIP device")
        need = self.byte_offset + tiled_bytes(self.ggml_type, self.n, self.k)
        if self.data.numel() < need:
            raise ValueError(f"GGUFWeight buffer holds {self.data.numel()} B, needs {need} B")
        if self.byte_offset % 16:
            raise ValueError(f"byteOffset {self.byte_offset} must be a multiple of 16")

    @property
    def row_bytes(self) -> int:
        return tile_row_bytes(self.ggml_type, self.k)

    @property
    def nbytes(self) -> int:
        return tiled_bytes(self.ggml_type, self.n, self.k)

    @property
    def type_name(self) -> str:
        return GGML_TYPE_NAMES[self.ggml_type]

    @property
    def device(self) -> torch.device:
        return self.data.device

    def ptr(self) -> int:
        return self.data.data_ptr() + self.byte_offset

    def rows(self, start: int, stop: int) -> "GGUFWeight":
        """Row-range view ``[start, stop)`` sharing storage.

        ``start`` must be a multiple of 16 (a tile boundary).  A view whose
        length is not a multiple of 16 keeps its last tile's trailing rows in
        place; kernels compute but never store or return them."""
        if not 0 <= start <= stop <= self.n:
            raise ValueError(f"row range [{start}, {stop}) outside [0, {self.n})")
        if start % TILE_ROWS:
            raise ValueError(f"row range must start on a multiple of {TILE_ROWS}, got {start}")
        return GGUFWeight(self.data, self.ggml_type, stop - start, self.k,
                          self.byte_offset + start * self.row_bytes)

    @classmethod
    def from_raw(cls, ggml_type: int, raw, n: int, k: int, device=None) -> "GGUFWeight":
        return repack_gguf_for_gpu(ggml_type, raw, n, k, device=device)

    def dequant(self) -> torch.Tensor:
        return dequant_ggml(self.ggml_type, self, self.n * self.k).view(self.n, self.k)


class LayerWeights:
    """Per-layer weight slots; ``<proj>_gg`` holds a GGUFWeight (forward-pass.ts:154-171)."""

    def __init__(self, **slots):
        self.__dict__.update(slots)

    def get(self, name, default=None):
        return self.__dict__.get(name, default)


def repack_gguf_for_gpu(ggml_type: int, data, n: int, k: Optional[int] = None,
                        device=None) -> GGUFWeight:
    """Raw GGUF bytes of an ``[n, k]`` tensor -> GGUFWeight in the row-tile layout.

    Mirrors repackGGUFForGPU (gguf-dequant.ts:809-840): ``repack(type, data, n)``
    with a single argument treats the data as one row of ``n`` elements; the
    byte length must match exactly (assertBytes, :678-680).
    """
    lib = _native.load_library()
    if k is None:
        n, k = 1, n
    check_kernel_type(ggml_type)
    raw = _as_device_u8(data, device)
    dev = raw.device
    out = torch.empty(tiled_bytes(ggml_type, n, k), dtype=torch.uint8, device=dev)
    with torch.cuda.device(dev):
        _native.check(lib.gguf_hip_repack(raw.data_ptr(), raw.numel(), ggml_type, n, k,
                                          out.data_ptr(), out.numel(), _stream(dev)), lib)
    return GGUFWeight(out, ggml_type, n, k)


def concat_rows(*weights: GGUFWeight) -> GGUFWeight:
    """Row-concatenate weights of one type and K (gate+up fusion, forward-pass.ts:740-791).

    Every weight but the last must have a multiple of 16 rows, so that the
    parts' tiles line up."""
    if not weights:
        raise ValueError("concat_rows needs at least one weight")
    t, k = weights[0].ggml_type, weights[0].k
    for w in weights:
        if w.ggml_type != t or w.k != k:
            raise ValueError("concat_rows: weights must share ggml type and K")
    for w in weights[:-1]:
        if w.n % TILE_ROWS:
            raise ValueError(f"concat_rows: all but the last weight need a multiple of "
                             f"{TILE_ROWS} rows, got {w.n}")
    parts = [w.data[w.byte_offset:w.byte_offset + w.nbytes] for w in weights]
    return GGUFWeight(torch.cat(parts), t, sum(w.n for w in weights), k)


def interleave_tiles(gate: GGUFWeight, up: GGUFWeight) -> GGUFWeight:
    """Gate and up weights with their 16-row tiles interleaved: tile 2m holds gate
    rows 16m..16m+15, tile 2m + 1 the same up rows.  A matmul over it computes
    the rows of the reference's gate+up concatenation (forward-pass.ts:740-791)
    in this order, and the SwiGLU epilogue of the fused decode kernel pairs
    them in one workgroup.  Both weights need the same type, K and a multiple
    of 16 rows."""
    if gate.ggml_type != up.ggml_type or gate.k != up.k or gate.n != up.n:
        raise ValueError("interleave_tiles: gate and up must share type and shape")
    if gate.n % TILE_ROWS:
        raise ValueError(f"interleave_tiles: rows must be a multiple of {TILE_ROWS}")
    tb = TILE_ROWS * gate.row_bytes
    nt = gate.n // TILE_ROWS
    g = gate.data[gate.byte_offset:gate.byte_offset + gate.nbytes].view(nt, tb)
    u = up.data[up.byte_offset:up.byte_offset + up.nbytes].view(nt, tb)
    return GGUFWeight(torch.stack([g, u], dim=1).reshape(-1), gate.ggml_type, 2 * gate.n, gate.k)


def split_interleaved(y: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """(gate, up) columns of a result ``[M, 2 * ffn]`` computed over ``interleave_tiles``."""
    m, n2 = y.shape
    v = y.view(m, n2 // (2 * TILE_ROWS), 2, TILE_ROWS)
    return v[:, :, 0, :].reshape(m, n2 // 2), v[:, :, 1, :].reshape(m, n2 // 2)


def dequant_ggml(ggml_type: int, data, n: int) -> torch.Tensor:
    """Dequantize ``n`` elements to f32 on the GPU (gguf-dequant.ts:844-868).

    ``data`` is a GGUFWeight (row-tile layout) or raw GGUF bytes (device or host).
    """
    lib = _native.load_library()
    check_kernel_type(ggml_type)
    if isinstance(data, GGUFWeight):
        if data.ggml_type != ggml_type or data.n * data.k != n:
            raise ValueError("dequant_ggml: type or element count does not match the weight")
        dev = data.device
        out = torch.empty(n, dtype=torch.float32, device=dev)
        with torch.cuda.device(dev):
            _native.check(lib.gguf_hip_dequant(data.ptr(), ggml_type, data.n, data.k,
                                               out.data_ptr(), data.k, _stream(dev)), lib)
        return out
    return dequant_raw(ggml_type, data, n)


def dequant_raw(ggml_type: int, data, n: int, device=None) -> torch.Tensor:
    """Dequantize raw GGUF bytes (any alignment) to f32 on the GPU."""
    lib = _native.load_library()
    raw = _as_device_u8(data, device)
    block, tsize, _ = ggml_type_traits(ggml_type)
    if n % block == 0 and raw.numel() != n // block * tsize:
        raise ValueError(f"[GGUF-dequant] byteLength {raw.numel()} != expected {n // block * tsize}")
    dev = raw.device
    out = torch.empty(n, dtype=torch.float32, device=dev)
    with torch.cuda.device(dev):
        _native.check(lib.gguf_hip_dequant_raw(raw.data_ptr(), ggml_type, n, out.data_ptr(),
                                               _stream(dev)), lib)
    return out


@dataclasses.dataclass
class QuantEmbedding:
    """A table of ``n`` raw GGUF rows of ``k`` elements resident in HBM.

    ``gather(ids)`` dequantizes the rows named by a device int64 tensor with
    one launch (``gguf_hip_get_rows``).  The reference keeps ``token_embd`` in
    host RAM as raw blocks and row-gathers + dequantizes each token on the CPU
    (webgpu/src/model/gguf-loader.ts:177-187, webgpu/src/engine/forward-pass.ts:2171-2186);
    with 288 GB of HBM the table stays on the device and the token id never
    leaves it, so a decode step that embeds its token can be graph-captured.
    An id outside ``[0, n)`` produces a row of NaN."""

    data: torch.Tensor   # uint8, raw GGUF bytes of the n rows
    ggml_type: int
    n: int
    k: int

    def __post_init__(self):
        check_kernel_type(self.ggml_type)
        if self.data.dtype != torch.uint8 or not self.data.is_cuda:
            raise ValueError("QuantEmbedding.data must be a uint8 tensor on a HIP device")
        need = self.n * raw_row_bytes(self.ggml_type, self.k)
        if self.data.numel() != need:
            raise ValueError(f"[GGUF] token table holds {self.data.numel()} B, expected {need}")

    @property
    def device(self) -> torch.device:
        return self.data.device

    def gather(self, ids: torch.Tensor, out: Optional[torch.Tensor] = None) -> torch.Tensor:
        """f32 ``[len(ids), k]`` rows (written into ``out`` when given)."""
        lib = _native.load_library()
        if ids.dtype != torch.int64 or ids.device != self.device:
            raise ValueError("QuantEmbedding.gather: ids must be int64 on the table's device")
        ids = ids.reshape(-1).contiguous()
        if out is None:
            out = torch.empty(ids.numel(), self.k, dtype=torch.float32, device=self.device)
        ldo = _row_stride(out, ids.numel(), self.k, "out")
        if out.dtype != torch.float32:
            raise ValueError("QuantEmbedding.gather: out must be float32")
        with torch.cuda.device(self.device):
            _native.check(lib.gguf_hip_get_rows(self.data.data_ptr(), self.ggml_type, self.n,
                                                self.k, ids.data_ptr(), ids.numel(),
                                                out.data_ptr(), ldo, _stream(self.device)), lib)
        return out


def _row_stride(t: torch.Tensor, rows: int, cols: int, name: str) -> int:
    if t.dim() == 1:
        if t.numel() < rows * cols:
            raise ValueError(f"{name} has {t.numel()} elements, needs {rows * cols}")
        return cols
    if t.dim() != 2 or t.stride(-1) != 1:
        raise ValueError(f"{name} must be 1-D or a 2-D tensor with unit column stride")
    if t.shape[0] < rows or t.shape[1] < cols:
        raise ValueError(f"{name} shape {tuple(t.shape)} smaller than [{rows}, {cols}]")
    return t.stride(0) if rows > 1 else max(t.stride(0), cols)


# Matmul workspaces.  Calls that share a workspace must not overlap (the
# split-K partial sums and the activation image), and calls on one stream
# are ordered, so there is one workspace per (device, stream): two streams of
# one device never share one.  It is allocated zero-filled once (its first
# 64 KB are reserved and stay zero).
# Under graph capture the key also carries the capture: the graph's workspace
# is allocated inside the capture (its zero fill is a kernel the graph replays
# ahead of the first use) and is never handed to eager calls, so replays and
# eager calls on the capturing stream do not share one; two graphs captured on
# one stream share theirs and must not be replayed concurrently.  Workspaces
# grow to the next power of two; an outgrown eager workspace is freed (its
# stream's later work is ordered after the calls that used it), an outgrown
# graph workspace is kept, since the graph still addresses it.
_WORKSPACES: dict = {}
_GRAPH_KEPT: list = []
_MIN_WORKSPACE = 1 << 20


def workspace_key(device_index: int, stream_handle: int, capturing: bool) -> tuple:
    """Key of the workspace a call uses: one per (device, stream), separate for
    calls made under graph capture."""
    return (int(device_index), int(stream_handle), bool(capturing))


def workspace_size(nbytes: int) -> int:
    """Bytes allocated for a request of ``nbytes``: the next power of two, at least 1 MiB."""
    return max(_MIN_WORKSPACE, 1 << max(0, int(nbytes) - 1).bit_length())


def matmul_workspace(dev: torch.device, nbytes: int) -> torch.Tensor:
    """The zero-initialised matmul workspace of the current stream of ``dev``
    (at least ``nbytes``)."""
    idx = dev.index if dev.index is not None else torch.cuda.current_device()
    stream = torch.cuda.current_stream(idx)
    capturing = torch.cuda.is_current_stream_capturing()
    key = workspace_key(idx, stream.cuda_stream, capturing)
    ws = _WORKSPACES.get(key)
    if ws is None or ws.numel() < nbytes:
        if ws is not None and capturing:
            _GRAPH_KEPT.append(ws)
        ws = torch.zeros(workspace_size(nbytes), dtype=torch.uint8, device=dev)
        _WORKSPACES[key] = ws
    return ws


def dispatch_matmul_gguf(a: torch.Tensor, gg: GGUFWeight, c: torch.Tensor, M: int, N: int,
                         K: int, label: str = "", io: Optional[dict] = None,
                         variant: int = _native.VARIANT_AUTO) -> None:
    """``C[M, N] = A[M, K] @ dequant(W)^T`` (forward-pass.ts:1496-1544).

    ``a``: f32 or f16 device tensor, ``c``: f32 device tensor (1-D or 2-D with
    unit column stride).  ``io = {"aOffset": bytes, "cOffset": bytes}`` selects
    windows of the buffers as the reference's MatmulIO does (offsets must be
    16-byte multiples here; the reference requires 256).
    """
    lib = _native.load_library()
    if gg.n != N or gg.k != K:
        raise ValueError(f'matmul_gguf "{label}": weight is [{gg.n}, {gg.k}], call asks [{N}, {K}]')
    if a.dtype not in _X_TYPES:
        raise ValueError(f'matmul_gguf "{label}": activations must be float32 or float16')
    if c.dtype != torch.float32:
        raise ValueError(f'matmul_gguf "{label}": output must be float32')
    if not (a.is_cuda and c.is_cuda) or a.device != gg.device or c.device != gg.device:
        raise ValueError(f'matmul_gguf "{label}": tensors must be on the weight\'s device')
    a_off = int((io or {}).get("aOffset", 0) or 0)
    c_off = int((io or {}).get("cOffset", 0) or 0)
    if a_off % 16 or c_off % 16:
        raise ValueError(f'matmul_gguf "{label}": io offsets must be multiples of 16 bytes')
    ldx = _row_stride(a, M, K, "A") if a_off == 0 else K
    ldy = _row_stride(c, M, N, "C") if c_off == 0 else N
    if a_off and a.numel() * a.element_size() < a_off + M * K * a.element_size():
        raise ValueError(f'matmul_gguf "{label}": A window out of range')
    if c_off and c.numel() * 4 < c_off + M * N * 4:
        raise ValueError(f'matmul_gguf "{label}": C window out of range')
    dev = gg.device
    x_type = _X_TYPES[a.dtype]
    # the split-K paths' workspace (activation image, partial sums of the K slices)
    need = _native.check(lib.gguf_hip_matmul_workspace(gg.ggml_type, x_type, N, K, M), lib)
    work = matmul_workspace(dev, need) if need > 0 else None
    with torch.cuda.device(dev):
        _native.check(lib.gguf_hip_matmul_ws(
            a.data_ptr() + a_off, x_type, ldx, gg.ptr(), gg.ggml_type, N, K,
            c.data_ptr() + c_off, ldy, M, variant, work.data_ptr() if work is not None else None,
            need, _stream(dev)), lib)


def dispatch_projection(input_buf: torch.Tensor, lw: LayerWeights, proj: str,
                        output_buf: torch.Tensor, M: int, N: int, K: int, label: str = "",
                        io: Optional[dict] = None) -> None:
    """Per-layer projection (forward-pass.ts:1576-1629): a ``<proj>_gg`` GGUF weight
    takes priority; an unquantized ``<proj>`` weight ``[N, K]`` (f32/f16/bf16) runs
    as a dense torch matmul, the reference's f32/BF16 branch (:1617-1627)."""
    gg = lw.get(f"{proj}_gg")
    if gg is not None:
        dispatch_matmul_gguf(input_buf, gg, output_buf, M, N, K, label, io)
        return
    w = lw.get(proj)
    if w is None:
        raise ValueError(f'dispatchProjection "{label}": layer has no weight "{proj}"')
    if io and (io.get("aOffset") or io.get("cOffset")):
        a = input_buf.view(-1)[io.get("aOffset", 0) // input_buf.element_size():]
        c = output_buf.view(-1)[io.get("cOffset", 0) // 4:]
    else:
        a, c = input_buf.view(-1), output_buf.view(-1)
    x = a[:M * K].view(M, K).to(w.dtype)
    c[:M * N].view(M, N).copy_(torch.matmul(x, w.t()).float())


def qlinear(x: torch.Tensor, w: GGUFWeight, out: Optional[torch.Tensor] = None,
            variant: int = _native.VARIANT_AUTO) -> torch.Tensor:
    """``y = x @ dequant(w)^T`` for ``x`` of shape ``[..., K]`` (f32/f16) -> f32 ``[..., N]``."""
    if x.shape[-1] != w.k:
        raise ValueError(f"qlinear: x has K={x.shape[-1]}, weight has K={w.k}")
    lead = x.shape[:-1]
    x2 = x.reshape(-1, w.k)
    if x2.stride(-1) != 1 or (x2.data_ptr() % 16) or (
            x2.shape[0] > 1 and (x2.stride(0) * x2.element_size()) % 16):
        x2 = x2.clone(memory_format=torch.contiguous_format)  # fresh, 16-byte aligned
    M = x2.shape[0]
    if out is None:
        out = torch.empty((M, w.n), dtype=torch.float32, device=w.device)
    y2 = out.view(M, w.n)
    dispatch_matmul_gguf(x2, w, y2, M, w.n, w.k, "qlinear", variant=variant)
    return out.view(*lead, w.n)
