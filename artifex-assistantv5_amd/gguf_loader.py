"""GGUF model loader: places a file's tensors in HBM for the quantized path.

Mirrors ``loadGGUFModel`` (``webgpu/src/model/gguf-loader.ts:166-460``):

* quantized matrices of a type the HIP kernels decode (``ggml.KERNEL_TYPES``:
  Q8_0, Q2_K - Q6_K, Q4_0, Q5_0, IQ4_NL, IQ4_XS, IQ2_XXS, IQ2_XS, IQ2_S,
  IQ3_XXS, IQ3_S, IQ1_M) are copied to the device and repacked there into the row-tile layout
  (``repackGGUFForGPU``, ``gguf-loader.ts:422-424``) -> ``GGUFWeight``;
* F32 tensors are uploaded as they are; F16 / BF16 tensors become f32 at load
  (``gguf-loader.ts:401-421``);
* ``token_embd.weight`` / ``per_layer_token_embd.weight`` are row-gather
  tables.  The reference keeps them in host RAM and dequantizes rows on the CPU
  (``gguf-loader.ts:177-187``); here they stay in HBM as raw GGUF rows
  (``QuantEmbedding``, gathered by a HIP kernel), or as f32 for F32/F16/BF16
  tables.  With tied embeddings (no ``output.weight``) ``token_embd`` is also
  repacked as a GGUFWeight for the LM head (``gguf-loader.ts:177,187``);
* ``rope_freqs.weight`` stays on the host (it is read, not dispatched);
* MoE expert slabs (``blk.N.ffn_{gate,up,down}_exps``) are not loaded: their
  tensor infos are returned in ``expert_tensors``, as the reference hands them
  to its CPU worker fleet (``gguf-loader.ts:100-106,262-270``); vision tensors
  (``v.*``, ``mm.*``), next-token-prediction blocks (``blk.L`` with
  ``L >= block_count - nextn_predict_layers``) and the dead K/V projections of
  KV-sharing layers are skipped (``gguf-loader.ts:188-227``).

Before any tensor is read, a pre-flight check rejects files holding types this
library cannot run (``gguf-loader.ts:229-256``), and an optional HBM budget is
checked against the planned device bytes (``plannedGPUBytes``, ``:115-124``).
Tensor bytes are read through a memory map in chunks of at most 128 MiB, each
checked for its length (``fetchTensorBytes``, ``:126-140``).
"""

from __future__ import annotations

import dataclasses
import mmap
import os
import re
import time
import warnings
from typing import Any, Callable, Dict, Optional, Union

import numpy as np
import torch

from .ggml import BF16, F16, F32, GGML_TYPE_NAMES, KERNEL_TYPES, raw_row_bytes, tiled_bytes
from .gguf_file import GGUFFile, GGUFTensorInfo, arch_kv, parse_gguf_path
from .linear import GGUFWeight, QuantEmbedding, repack_gguf_for_gpu

MAX_CHUNK = 128 * 1024 * 1024                     # gguf-loader.ts:99
EXPERT_RE = re.compile(r"^blk\.\d+\.ffn_(gate|up|down)_exps\.weight$")   # :105
FUSED_EXPERT_RE = re.compile(r"^blk\.\d+\.ffn_gate_up_exps\.weight$")    # :106
BLK_RE = re.compile(r"^blk\.(\d+)\.")                                     # :108
DEAD_KV_RE = re.compile(r"^blk\.(\d+)\.(attn_k|attn_v|attn_k_norm)\.weight$")  # :109
ROW_GATHER_NAMES = ("token_embd.weight", "per_layer_token_embd.weight")
HOST_NAMES = ("rope_freqs.weight",)
SUPPORTED_TYPES = frozenset((F32, F16, BF16) + tuple(KERNEL_TYPES))

# A transform of a quantized matrix's raw rows before the repack:
# (tensor info, device uint8 [rows, row_bytes]) -> same shape.
RawTransform = Callable[[GGUFTensorInfo, torch.Tensor], torch.Tensor]


@dataclasses.dataclass
class GGUFTensorGPU:
    """One placed tensor (``GGUFTensorGPU``, gguf-loader.ts:33-46)."""
    name: str
    data: Union[GGUFWeight, torch.Tensor]   # GGUFWeight when quantized, else f32
    shape: list                              # [out, in] for matrices
    dtype: str                               # GGML type name of the file's tensor
    ggml_type: int
    byte_length: int                         # device bytes
    element_count: int
    is_quantized: bool


@dataclasses.dataclass
class LoadedGGUFModel:
    """``LoadedGGUFModel`` (gguf-loader.ts:66-89) for one device."""
    path: str
    file: GGUFFile
    tensors: Dict[str, GGUFTensorGPU]
    row_tables: Dict[str, Union[QuantEmbedding, torch.Tensor]]   # the reference's cpuTensors
    host_tensors: Dict[str, np.ndarray]
    expert_tensors: Dict[str, GGUFTensorInfo]
    expert_bytes: int
    total_gpu_bytes: int
    tensor_count: int
    load_time_ms: float


def planned_gpu_bytes(t: GGUFTensorInfo) -> int:
    """Device bytes of a tensor after placement (plannedGPUBytes, gguf-loader.ts:115-124)."""
    if t.ggml_type in KERNEL_TYPES:
        rows = t.element_count // t.ne[0] if t.ne else 1
        return tiled_bytes(t.ggml_type, rows, t.ne[0])
    if t.ggml_type in (F16, BF16):
        return t.element_count * 4
    return t.byte_length


def _mapped(path: str):
    with open(path, "rb") as f:
        return mmap.mmap(f.fileno(), 0, access=mmap.ACCESS_READ)


def read_tensor_to_device(mm, t: GGUFTensorInfo, device) -> torch.Tensor:
    """The tensor's raw bytes as a device uint8 tensor, copied in <= 128 MiB chunks
    with a length check on every chunk (fetchTensorBytes, gguf-loader.ts:126-140)."""
    out = torch.empty(t.byte_length, dtype=torch.uint8, device=device)
    got = 0
    while got < t.byte_length:
        n = min(MAX_CHUNK, t.byte_length - got)
        start = t.offset + got
        have = max(0, min(n, len(mm) - start))
        if have != n:
            raise ValueError(f"[GGUF] Short range read at {start}: got {have}, want {n}")
        part = np.frombuffer(mm, dtype=np.uint8, count=n, offset=start)
        with warnings.catch_warnings():   # read-only map: the copy only reads it
            warnings.simplefilter("ignore", UserWarning)
            out[got:got + n].copy_(torch.from_numpy(part))
        got += n
    return out


def _to_f32(raw: torch.Tensor, t: GGUFTensorInfo) -> torch.Tensor:
    if t.ggml_type == F32:
        v = raw.view(torch.float32)
    elif t.ggml_type == F16:
        v = raw.view(torch.float16).float()
    else:
        v = raw.view(torch.bfloat16).float()
    return v.reshape(t.shape) if t.shape else v


def load_gguf_model(path: str, device="cuda", on_progress: Optional[Callable[[str], Any]] = None,
                    vram_budget_bytes: Optional[int] = None,
                    raw_transform: Optional[RawTransform] = None) -> LoadedGGUFModel:
    """Parse ``path`` and place its tensors on ``device``.

    ``raw_transform`` may rewrite a quantized matrix's raw rows (a row
    permutation, for instance) before it is repacked."""
    t0 = time.perf_counter()
    dev = torch.device(device)
    file = parse_gguf_path(path)
    say = on_progress or (lambda msg: None)

    tied = "output.weight" not in file.tensors
    also_gpu = {"token_embd.weight"} if tied else set()
    n_layers = arch_kv(file, "block_count") - arch_kv(file, "nextn_predict_layers", 0)

    def is_mtp(name: str) -> bool:
        m = BLK_RE.match(name)
        return m is not None and int(m.group(1)) >= n_layers

    shared_kv = arch_kv(file, "attention.shared_kv_layers", 0)
    kv_from = n_layers - shared_kv

    def is_dead_kv(name: str) -> bool:
        if shared_kv <= 0:
            return False
        m = DEAD_KV_RE.match(name)
        return m is not None and int(m.group(1)) >= kv_from

    def is_vision(name: str) -> bool:
        return name.startswith("v.") or name.startswith("mm.")

    # pre-flight: every tensor that will be placed must have a type this library runs
    unsupported: Dict[str, int] = {}
    experts: Dict[str, GGUFTensorInfo] = {}
    for t in file.tensors.values():
        if FUSED_EXPERT_RE.match(t.name):
            raise ValueError(f'[GGUF] "{t.name}": fused gate+up expert tensors unsupported — '
                             "expected split ffn_gate_exps/ffn_up_exps")
        if EXPERT_RE.match(t.name):
            experts[t.name] = t
            continue
        if is_vision(t.name) or is_dead_kv(t.name) or is_mtp(t.name) or t.name in HOST_NAMES:
            continue
        if t.ggml_type not in SUPPORTED_TYPES:
            unsupported[t.type_name] = unsupported.get(t.type_name, 0) + 1
    if unsupported:
        lst = ", ".join(f"{n} ({c} tensors)" for n, c in unsupported.items())
        names = ", ".join(GGML_TYPE_NAMES[t] for t in sorted(KERNEL_TYPES))
        raise ValueError(f"This GGUF uses quantization the HIP engine can't run yet: {lst}. "
                         f"Supported: {names} (and F16/F32/BF16).")

    placed = [t for t in file.tensors.values()
              if not (t.name in experts or is_vision(t.name) or is_dead_kv(t.name)
                      or is_mtp(t.name))]
    if vram_budget_bytes is not None:
        planned = sum(planned_gpu_bytes(t) for t in placed if t.name not in HOST_NAMES)
        planned += sum(planned_gpu_bytes(file.tensors[n]) for n in also_gpu if n in file.tensors)
        if planned > vram_budget_bytes:
            raise ValueError(f"[GGUF] model needs {planned / 1e9:.2f} GB of device memory, "
                             f"budget is {vram_budget_bytes / 1e9:.2f} GB")

    mm = _mapped(path)
    tensors: Dict[str, GGUFTensorGPU] = {}
    row_tables: Dict[str, Union[QuantEmbedding, torch.Tensor]] = {}
    host: Dict[str, np.ndarray] = {}
    total = 0
    try:
        for i, t in enumerate(placed):
            say(f"[{i + 1}/{len(placed)}] {t.name} ({t.type_name}, {t.byte_length / 1e6:.1f} MB)")
            if t.name in HOST_NAMES:
                host[t.name] = np.frombuffer(mm[t.offset:t.offset + t.byte_length],
                                             dtype=np.uint8).copy()
                continue
            raw = read_tensor_to_device(mm, t, dev)
            k = t.ne[0] if t.ne else 1
            rows = t.element_count // k if k else 0
            gather = t.name in ROW_GATHER_NAMES
            if gather:
                if t.ggml_type in KERNEL_TYPES:
                    row_tables[t.name] = QuantEmbedding(raw, t.ggml_type, rows, k)
                else:
                    row_tables[t.name] = _to_f32(raw, t).reshape(rows, k)
                total += raw.numel() if t.ggml_type in KERNEL_TYPES else rows * k * 4
                if t.name not in also_gpu:
                    continue
            if t.ggml_type in KERNEL_TYPES:
                if raw_transform is not None:
                    raw = raw_transform(t, raw.view(rows, raw_row_bytes(t.ggml_type, k)))
                    raw = raw.reshape(-1)
                w = repack_gguf_for_gpu(t.ggml_type, raw, rows, k, device=dev)
                del raw
                tensors[t.name] = GGUFTensorGPU(t.name, w, t.shape, t.type_name, t.ggml_type,
                                                w.nbytes, t.element_count, True)
                total += w.nbytes
            else:
                v = _to_f32(raw, t)
                tensors[t.name] = GGUFTensorGPU(t.name, v, t.shape, t.type_name, t.ggml_type,
                                                v.numel() * 4, t.element_count, False)
                total += v.numel() * 4
    finally:
        mm.close()
    torch.cuda.synchronize(dev)
    return LoadedGGUFModel(
        path=path, file=file, tensors=tensors, row_tables=row_tables, host_tensors=host,
        expert_tensors=experts, expert_bytes=sum(t.byte_length for t in experts.values()),
        total_gpu_bytes=total, tensor_count=file.tensor_count,
        load_time_ms=(time.perf_counter() - t0) * 1000.0)
