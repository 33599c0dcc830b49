"""`GLiNERDecideClassifier` (DeBERTa.swift:152-447) on the HIP library.

The Swift public surface is kept: a constructor with the same feature flags,
`classify(input, collect_profile=False) -> InferenceResult`, `DecisionInput`
with the four arrays, and `InferenceResult{logits, wall_nanoseconds, events}`.
"""

from __future__ import annotations

import ctypes as C
import time
from dataclasses import dataclass, field
from pathlib import Path

import numpy as np
import torch

from . import _native as N
from .config import DeBERTaV2Configuration
from .decode import row_extents
from .device import require_gpu, stream_handle
from .weights import WeightStore


@dataclass(frozen=True)
class ProfileEvent:  # DeBERTa.swift:7-12
    name: str
    nanoseconds: int

    @property
    def milliseconds(self) -> float:
        return self.nanoseconds / 1e6


@dataclass
class InferenceResult:  # DeBERTa.swift:14-20
    logits: torch.Tensor  # [B, Hh, O] fp16 on the GPU
    wall_nanoseconds: int
    events: list = field(default_factory=list)

    @property
    def wall_milliseconds(self) -> float:
        return self.wall_nanoseconds / 1e6


@dataclass
class DecisionInput:  # DeBERTa.swift:22-58
    """input_ids [B, L] int, attention_mask [B, L] (1 = token), marker_indices
    [B, Hh, O] int, marker_mask [B, Hh, O].  Accepts numpy arrays or torch
    tensors; `to_device` returns the dtypes the library takes (int32, fp16,
    int32, fp32) on the GPU."""

    input_ids: object
    attention_mask: object
    marker_indices: object
    marker_mask: object

    @classmethod
    def from_safetensors(cls, path: str | Path) -> "DecisionInput":  # DecisionInput(url:), :40-57
        from safetensors.numpy import load_file
        arrays = load_file(str(path))
        missing = [k for k in ("input_ids", "attention_mask", "marker_indices", "marker_mask") if k not in arrays]
        if missing:
            raise N.GlinerDecideError(N.GD_ERR_INVALID_ARGUMENT,
                                      "Input safetensors must contain input_ids, attention_mask, marker_indices, "
                                      "and marker_mask")
        return cls(arrays["input_ids"], arrays["attention_mask"], arrays["marker_indices"], arrays["marker_mask"])

    @property
    def shape(self):
        B, L = tuple(self.input_ids.shape)
        _, Hh, O = tuple(self.marker_indices.shape)
        return B, L, Hh, O

    def to_device(self, device=None):
        device = device or require_gpu()

        def conv(x, dtype):
            t = x if isinstance(x, torch.Tensor) else torch.from_numpy(np.ascontiguousarray(x))
            return t.to(device=device, dtype=dtype).contiguous()

        return (conv(self.input_ids, torch.int32), conv(self.attention_mask, torch.float16),
                conv(self.marker_indices, torch.int32), conv(self.marker_mask, torch.float32))


class GLiNERDecideClassifier:
    """Mirror of `GLiNERDecideClassifier.init` (DeBERTa.swift:188-196).

    weights: a WeightStore, a path to an fp16 safetensors file, or a dict of
    numpy arrays keyed like the checkpoint.  Every flag reproduces the
    reference graph it selects (DeBERTa.swift:322-464): use_fused_kernels keeps
    the residual sum in fp32 (FusedKernels residual LN);
    use_fast_attention=False takes the explicit-score path (:397-409);
    use_custom_relative_kernel uses the relative-bias Metal kernel's fp32 bias
    as the attention mask (:357-372, 383-385); use_fused_attention_kernel the
    fused-attention Metal kernel's fp32 score (:337-354); either of the last
    two also switches the residual LNs to the fp32 sum, as the reference does
    whenever it holds a FusedKernels instance.  use_compiled_graph replays a
    captured hipGraph per input shape (MLX `compile`).  full_rows (no
    counterpart in the reference) makes classify compute every position; by
    default each row's attention stops at its extent (last unmasked or
    marker-read position + 1), which leaves the logits unchanged.
    """

    def __init__(self, weights, configuration: DeBERTaV2Configuration | None = None, use_fused_kernels: bool = False,
                 use_compiled_graph: bool = False, use_fast_attention: bool = True,
                 use_custom_relative_kernel: bool = False, use_fused_attention_kernel: bool = False,
                 full_rows: bool = False):
        require_gpu()
        self._lib = N.lib()
        self.configuration = configuration or DeBERTaV2Configuration.default()
        if isinstance(weights, WeightStore):
            store = weights
        elif isinstance(weights, (str, Path)):
            store = WeightStore(url=weights)
        else:
            store = WeightStore(arrays=weights)
        flags = 0
        if use_fused_kernels:
            flags |= N.GD_USE_FUSED_KERNELS
        if use_compiled_graph:
            flags |= N.GD_USE_COMPILED_GRAPH
        if not use_fast_attention:
            flags |= N.GD_USE_GENERIC_ATTENTION
        if use_custom_relative_kernel:
            flags |= N.GD_USE_CUSTOM_RELATIVE_KERNEL
        if use_fused_attention_kernel:
            flags |= N.GD_USE_FUSED_ATTENTION_KERNEL
        if full_rows:
            flags |= N.GD_FULL_ROWS
        cfg = self.configuration.to_native()
        h = C.c_void_p()
        N.check(self._lib.gd_classifier_create(C.byref(h), store.handle, C.byref(cfg), flags, stream_handle()))
        self._h = h
        self.use_fused_kernels = use_fused_kernels
        self.use_compiled_graph = use_compiled_graph
        self.use_fast_attention = use_fast_attention
        self.use_custom_relative_kernel = use_custom_relative_kernel
        self.use_fused_attention_kernel = use_fused_attention_kernel
        self.full_rows = full_rows

    @property
    def device_bytes(self) -> int:
        return int(self._lib.gd_classifier_device_bytes(self._h))

    def reserve(self, batch: int, seq_len: int, max_heads: int, max_options: int) -> None:
        N.check(self._lib.gd_classifier_reserve(self._h, batch, seq_len, max_heads, max_options))

    def classify_device(self, ids: torch.Tensor, mask: torch.Tensor, markers: torch.Tensor, marker_mask: torch.Tensor,
                        out: torch.Tensor | None = None, total_tokens: int | None = None) -> torch.Tensor:
        """Enqueues the forward on the current stream; inputs already on the GPU
        with the library dtypes (int32, fp16, int32, fp32).  No sync.  With
        total_tokens (the sum of `row_extents`) the forward runs on packed
        rows (gd_classifier_classify_packed)."""
        B, L = ids.shape
        _, Hh, O = markers.shape
        if out is None:
            out = torch.empty((B, Hh, O), dtype=torch.float16, device=ids.device)
        if total_tokens is None:
            N.check(self._lib.gd_classifier_classify(self._h, ids.data_ptr(), mask.data_ptr(), markers.data_ptr(),
                                                     marker_mask.data_ptr(), B, L, Hh, O, out.data_ptr(),
                                                     stream_handle()))
        else:
            N.check(self._lib.gd_classifier_classify_packed(self._h, ids.data_ptr(), mask.data_ptr(),
                                                            markers.data_ptr(), marker_mask.data_ptr(), B, L, Hh, O,
                                                            int(total_tokens), out.data_ptr(), stream_handle()))
        return out

    def classify(self, inp: DecisionInput, collect_profile: bool = False) -> InferenceResult:
        """`classify(_:collectProfile:)` (DeBERTa.swift:244-272): runs the
        forward and synchronises (MLX `eval`).  Host-array inputs run on packed
        rows (their extents are known on the host) unless full_rows was set;
        tensors already on the GPU run padded."""
        total = None
        if not self.full_rows and not collect_profile and not isinstance(inp.attention_mask, torch.Tensor):
            total = int(row_extents(inp.attention_mask, inp.marker_indices, inp.marker_mask).sum())
        ids, mask, markers, mmask = inp.to_device()
        B, L, Hh, O = inp.shape
        out = torch.empty((B, Hh, O), dtype=torch.float16, device=ids.device)
        start = time.perf_counter_ns()
        events = []
        if collect_profile:
            cap = 8 + 4 * self.configuration.num_hidden_layers
            arr = (N.GdProfileEvent * cap)()
            n = C.c_int32(0)
            N.check(self._lib.gd_classifier_classify_profiled(self._h, ids.data_ptr(), mask.data_ptr(),
                                                              markers.data_ptr(), mmask.data_ptr(), B, L, Hh, O,
                                                              out.data_ptr(), arr, cap, C.byref(n), stream_handle()))
            events = [ProfileEvent(arr[i].name.decode(), int(arr[i].milliseconds * 1e6)) for i in range(n.value)]
        else:
            self.classify_device(ids, mask, markers, mmask, out, total_tokens=total)
        torch.cuda.current_stream().synchronize()
        return InferenceResult(out, time.perf_counter_ns() - start, events)

    def encode(self, inp_or_ids, attention_mask=None, num_layers: int = -1) -> torch.Tensor:
        """Final hidden states [B, L, C] fp16 after `num_layers` layers."""
        if isinstance(inp_or_ids, DecisionInput):
            ids, mask, _, _ = inp_or_ids.to_device()
        else:
            dev = require_gpu()
            ids = torch.as_tensor(inp_or_ids).to(dev, torch.int32).contiguous()
            mask = torch.as_tensor(attention_mask).to(dev, torch.float16).contiguous()
        B, L = ids.shape
        out = torch.empty((B, L, self.configuration.hidden_size), dtype=torch.float16, device=ids.device)
        N.check(self._lib.gd_classifier_encode(self._h, ids.data_ptr(), mask.data_ptr(), B, L, num_layers,
                                               out.data_ptr(), stream_handle()))
        return out

    def layer_forward(self, layer_index: int, hidden: torch.Tensor, attention_mask: torch.Tensor) -> torch.Tensor:
        """One encoder layer (DeBERTa.swift:296-428) on hidden states [B, L, C] fp16."""
        hidden = hidden.to(torch.float16).contiguous()
        mask = attention_mask.to(device=hidden.device, dtype=torch.float16).contiguous()
        B, L, _ = hidden.shape
        out = torch.empty_like(hidden)
        N.check(self._lib.gd_classifier_layer_forward(self._h, layer_index, hidden.data_ptr(), mask.data_ptr(), B, L,
                                                      out.data_ptr(), stream_handle()))
        return out

    def check_device_errors(self) -> None:
        N.check(self._lib.gd_classifier_check_device_errors(self._h, stream_handle()))

    def close(self) -> None:
        if getattr(self, "_h", None):
            self._lib.gd_classifier_destroy(self._h)
            self._h = C.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
