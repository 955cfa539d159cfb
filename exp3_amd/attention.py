"""Transformers attention backend: dense, V1 and mean-corrected sparse prefill on MI355X.

Drop-in for the reference ``attention.py``: same ``METHODS``, the same
``AttentionBackend`` constructor, ``configure``, ``forward`` signature, stage
names, profiling and capture hooks, and the same registration as transformers'
``"sdpa"`` attention function (attention.py:57). Prefill of the sparse methods
runs entirely in gfx950 HIP kernels:

  descriptor  spx_block_pool           bf16 mean K, fp32 descriptors, K / V tiles
  selector    spx_v1_route             V1 score + normalise + threshold selection
              spx_selector_scores      (mean_balanced / cgf_mean / dispersion_mean)
  indices     spx_protected_selection  (new selectors; V1 selection is fused above)
  mean        spx_tile_mean_query +    rescue-token choice (rescue methods only)
              spx_rescue_choice
  exact       spx_exact_attention      block-sparse flash attention
              spx_sparse_attention_mean  same, with the mean tail and the
                                         logaddexp merge fused in (mean methods)
              spx_sparse_attention_rescue  same, with the rescue tail fused in

so the reference's separate "merge" stage (and, for the mean methods, its "mean"
stage) takes no time here and is reported as 0 ms. Dense prefill and every decode step use
``F.scaled_dot_product_attention`` exactly as the reference does
(attention.py:179-189); ``dense_impl="hip"`` routes dense prefill through the
HIP kernel with implicit all-causal block lists instead.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F

from . import _lib, kernels
from .kernels import BlockDescriptors
from .upstream import flashprefill_native_forward as upstream

try:  # transformers is optional: the backend also runs standalone
    from transformers.modeling_utils import ALL_ATTENTION_FUNCTIONS
except Exception:  # pragma: no cover - depends on the environment
    ALL_ATTENTION_FUNCTIONS = None

METHODS = (
    "dense",
    "fp_v1",
    "mean_native",
    "mean_balanced",
    "cgf_mean",
    "dispersion_mean",
    "fp_v1_rescue",
    "fp_v1_rescue_v2",
)
V1_ROUTED_METHODS = {"fp_v1", "mean_native", "fp_v1_rescue", "fp_v1_rescue_v2"}
RESCUE_METHODS = {"fp_v1_rescue", "fp_v1_rescue_v2"}
MEAN_METHODS = {
    "mean_native",
    "mean_balanced",
    "cgf_mean",
    "dispersion_mean",
}
STAGE_NAMES = ("descriptor", "selector", "indices", "exact", "mean", "merge", "attention")


def _blocks(sequence: int, block_size: int) -> int:
    return (sequence + block_size - 1) // block_size


class AttentionBackend:
    """Reference: attention.py:37-369."""

    def __init__(
        self,
        alpha: float = 0.08,
        sink_blocks: int = 2,
        window_blocks: int = 4,
        last_full_blocks: int = 2,
        block_size: int = 128,
        selector_chunk_tiles: int = 8,
        register: bool = True,
        dense_impl: str = "sdpa",
    ):
        if dense_impl not in ("sdpa", "hip"):
            raise ValueError(f"dense_impl must be 'sdpa' or 'hip', got {dense_impl!r}")
        self.method = "dense"
        self.alpha = alpha
        self.sink_blocks = sink_blocks
        self.window_blocks = window_blocks
        self.last_full_blocks = last_full_blocks
        self.block_size = block_size
        self.selector_chunk_tiles = selector_chunk_tiles
        self.dense_impl = dense_impl
        self.record = False
        self.profile_records = []
        self.capture_callback = None
        # When a list, every attention-kernel launch appends its (start, end)
        # torch.cuda.Event pair, recorded on the launch stream (benchmarks).
        self.kernel_events = None
        if register and ALL_ATTENTION_FUNCTIONS is not None:
            ALL_ATTENTION_FUNCTIONS["sdpa"] = self.forward

    def configure(self, method: str, alpha: float | None = None):
        if method not in METHODS:
            raise ValueError(f"unknown method {method!r}; choose from {METHODS}")
        self.method = method
        if alpha is not None:
            self.alpha = alpha

    def _stage(self, record, name, function):
        if not self.record:
            return function()
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        start.record()
        result = function()
        end.record()
        record["events"][name] = (start, end)
        return result

    # ------------------------------------------------------------ pooling

    def _pool(self, k, v, want_kbar: bool, want_descriptors: bool, want_tiles: bool):
        """One spx_block_pool launch -> (bf16 mean K, descriptors, (key tiles,
        value tiles))."""
        device = _lib.require_gpu(k, v)
        batch, sequence, kv_heads, head_dim = k.shape
        blocks = _blocks(sequence, self.block_size)
        kbar = torch.empty(batch, blocks, kv_heads, head_dim, dtype=torch.bfloat16,
                           device=device) if want_kbar else None
        desc = kernels.empty_descriptors(batch, blocks, kv_heads, head_dim, device) \
            if want_descriptors else None
        tiles = (torch.empty(batch, kv_heads, blocks, self.block_size, head_dim,
                             dtype=torch.bfloat16, device=device),
                 torch.empty(batch, kv_heads, blocks, head_dim, self.block_size,
                             dtype=torch.bfloat16, device=device)) if want_tiles else None
        _lib.call(
            "spx_block_pool", _lib.ptr(k), _lib.strides(k), _lib.ptr(v), _lib.strides(v),
            batch, sequence, kv_heads, head_dim, self.block_size, _lib.ptr(kbar),
            _lib.ptr(desc.mean_k if desc else None), _lib.ptr(desc.mean_v if desc else None),
            _lib.ptr(desc.var_k if desc else None), _lib.ptr(desc.sigma_v if desc else None),
            _lib.ptr(desc.counts if desc else None), _lib.ptr(tiles[0] if tiles else None),
            _lib.ptr(tiles[1] if tiles else None), _lib.stream(device))
        return kbar, desc, tiles

    # ---------------------------------------------------------- selection

    def _route_v1(self, q, k, v, scale, record, want_descriptors, want_tiles,
                  want_scores=False):
        kbar, descriptors, tiles = self._stage(
            record, "descriptor",
            lambda: self._pool(k, v, True, want_descriptors, want_tiles))
        batch, sequence, q_heads, head_dim = q.shape
        blocks = kbar.shape[1]
        device = q.device
        scores = torch.empty(batch, blocks, blocks, q_heads, dtype=torch.float32,
                             device=device) if want_scores else None
        indices = torch.empty(batch, blocks, blocks, q_heads, dtype=torch.int64, device=device)
        counts = torch.empty(batch, blocks, q_heads, dtype=torch.int32, device=device)
        selected = torch.empty(batch, blocks, blocks, q_heads, dtype=torch.bool, device=device)

        def route():
            _lib.call(
                "spx_v1_route", _lib.ptr(q), _lib.strides(q), _lib.ptr(kbar), _lib.strides(kbar),
                batch, sequence, q_heads, k.shape[2], head_dim, self.block_size, float(scale),
                float(self.alpha), int(self.sink_blocks), int(self.window_blocks),
                int(self.last_full_blocks), _lib.ptr(scores), _lib.ptr(indices),
                _lib.ptr(counts), _lib.ptr(selected), _lib.stream(device))

        self._stage(record, "selector", route)
        return kbar, descriptors, tiles, scores, indices, counts, selected

    def _v1_selection(self, q, k, scale, record, descriptors_needed, return_auxiliary=False):
        """Reference attention.py:77-108: descriptors (fp32 only when a value
        tensor is given) + bf16 mean K -> V1 scores -> selection -> mask."""
        q = _lib.kernel_view(q)
        k = _lib.kernel_view(k)
        v = descriptors_needed if isinstance(descriptors_needed, torch.Tensor) else None
        if v is not None:
            v = _lib.kernel_view(v)
        kbar, descriptors, _, scores, indices, counts, selected = self._route_v1(
            q, k, v if v is not None else k, scale, record, v is not None, False,
            want_scores=return_auxiliary)
        if return_auxiliary:
            return descriptors, kbar, scores, indices, counts, selected
        return descriptors, indices, counts, selected

    def _new_selection(self, q, k, v, scale, record, want_tiles=False):
        """Reference attention.py:110-152 (plus the attention tiles of the pooling pass)."""
        _, descriptors, tiles = self._stage(
            record, "descriptor", lambda: self._pool(k, v, False, True, want_tiles))
        batch, sequence, q_heads, _ = q.shape
        blocks = descriptors.mean_k.shape[1]
        if self.alpha == 0:
            scores = torch.zeros(batch, blocks, blocks, q_heads, dtype=torch.float32,
                                 device=q.device)
        else:
            scores = self._stage(
                record, "selector",
                lambda: kernels.selector_scores(q, descriptors, scale, self.method,
                                                self.block_size, self.selector_chunk_tiles))
        indices = torch.empty(batch, blocks, blocks, q_heads, dtype=torch.int64, device=q.device)
        counts = torch.empty(batch, blocks, q_heads, dtype=torch.int32, device=q.device)
        selected = self._stage(
            record, "indices",
            lambda: kernels.protected_selection(scores, self.alpha, self.sink_blocks,
                                                self.window_blocks, self.last_full_blocks,
                                                indices, counts))
        return descriptors, tiles, indices, counts, selected

    # --------------------------------------------------------- attention

    def _attention(self, q, k, tiles, indices, counts, scale, descriptors: BlockDescriptors | None,
                   rescue=None, want_lse=True):
        """One attention-kernel launch: exact blocks, plus the block-mean tail
        (``descriptors``) or the rescue tail (``rescue`` = (choice, remainder,
        descriptors-or-None, v)) in the same online softmax. Returns (output, lse);
        lse is None when not wanted (the layer discards it, and the kernel then
        skips its stores)."""
        device = q.device
        batch, sequence, q_heads, head_dim = q.shape
        output = torch.empty(batch, sequence, q_heads, head_dim, dtype=q.dtype, device=device)
        lse = (torch.empty(batch, sequence, q_heads, dtype=torch.float32, device=device)
               if want_lse else None)
        common_head = (_lib.ptr(q), _lib.strides(q), _lib.ptr(tiles[0]), _lib.ptr(tiles[1]),
                       _lib.ptr(indices), _lib.strides(indices), _lib.ptr(counts),
                       _lib.strides(counts))
        # zeroed counters of the kernel's persistent grid (work items taken in turn)
        queue = torch.zeros(_lib.WORK_QUEUE_INTS, dtype=torch.int32, device=device)
        common_tail = (batch, sequence, q_heads, k.shape[2], head_dim, self.block_size,
                       float(scale), _lib.ptr(output), _lib.strides(output), _lib.ptr(lse),
                       _lib.strides(lse), _lib.ptr(queue), _lib.stream(device))
        if head_dim in upstream._ATTENTION_CONFIGS:   # what attention_tile_sizes() reports
            upstream._flash_forward.best_config = upstream._ATTENTION_CONFIGS[head_dim]
        events = None
        if self.kernel_events is not None:
            events = (torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
            events[0].record()
        if rescue is not None:
            choice, remainder, rdesc, values = rescue
            _lib.call("spx_sparse_attention_rescue", *common_head, _lib.ptr(choice),
                      _lib.ptr(values), _lib.strides(values),
                      _lib.ptr(rdesc.mean_k if rdesc else None),
                      _lib.ptr(rdesc.mean_v if rdesc else None), int(remainder), *common_tail)
        elif descriptors is None:
            _lib.call("spx_exact_attention", *common_head, *common_tail)
        else:
            _lib.call("spx_sparse_attention_mean", *common_head, _lib.ptr(descriptors.mean_k),
                      _lib.ptr(descriptors.mean_v), _lib.ptr(descriptors.counts), *common_tail)
        if events is not None:
            events[1].record()
            self.kernel_events.append(events)
        return output, lse

    def _dense_hip(self, q, k, v, scale):
        _, _, tiles = self._pool(k, v, False, False, True)
        return self._attention(q, k, tiles, None, None, scale, None, want_lse=False)

    def forward(
        self,
        module,
        query,
        key,
        value,
        attention_mask,
        scaling,
        dropout=0.0,
        **kwargs,
    ):
        """Reference attention.py:154-339. query [B, Hq, S, D], key / value
        [B, Hkv, S, D] -> (output [B, S, Hq, D], None)."""
        record = {
            "layer": getattr(module, "layer_idx", None),
            "method": self.method,
            "events": {},
            "accounting": None,
        }
        overall_start = overall_end = None
        if self.record:
            overall_start = torch.cuda.Event(enable_timing=True)
            overall_end = torch.cuda.Event(enable_timing=True)
            overall_start.record()

        is_prefill = query.shape[2] == key.shape[2]
        if (self.method == "dense" and self.dense_impl == "sdpa") or not is_prefill:
            output = F.scaled_dot_product_attention(
                query, key, value, attn_mask=None, dropout_p=0.0, is_causal=is_prefill,
                scale=scaling, enable_gqa=True,
            ).transpose(1, 2).contiguous()
            if self.record and is_prefill:
                record["accounting"] = self._dense_accounting(query)
        elif self.method == "dense":
            q = _lib.kernel_view(query.transpose(1, 2))
            k = _lib.kernel_view(key.transpose(1, 2))
            v = _lib.kernel_view(value.transpose(1, 2))
            output, _ = self._stage(record, "exact", lambda: self._dense_hip(q, k, v, float(scaling)))
            if self.record:
                record["accounting"] = self._dense_accounting(query)
        else:
            _lib.require_gpu(query, key, value)
            q = _lib.kernel_view(query.transpose(1, 2))
            k = _lib.kernel_view(key.transpose(1, 2))
            v = _lib.kernel_view(value.transpose(1, 2))
            scale = float(scaling)
            capture_v1 = self.capture_callback is not None and self.method == "fp_v1"
            if self.method in V1_ROUTED_METHODS:
                kbar, descriptors, tiles, scores, indices, counts, selected = self._route_v1(
                    q, k, v, scale, record,
                    self.method in ("mean_native", "fp_v1_rescue_v2"), True,
                    want_scores=capture_v1)
            else:
                descriptors, tiles, indices, counts, selected = self._new_selection(
                    q, k, v, scale, record, want_tiles=True)
                kbar = scores = None

            if capture_v1:
                self.capture_callback(
                    layer=int(module.layer_idx), q=q, k=k, v=v, mean_k=kbar, scores=scores,
                    indices=indices, counts=counts, selected=selected, scale=scale)

            mean_desc = descriptors if self.method in MEAN_METHODS else None
            rescue = None
            if self.method in RESCUE_METHODS:
                # the rescue-token choice is timed as the "mean" stage (the non-exact
                # tail path of the profile schema, attention.py:306-307); the tail
                # itself runs inside the attention kernel
                choice = self._stage(
                    record, "mean",
                    lambda: kernels.rescue_choice(q, tiles[0], self.block_size))
                rescue = (choice, self.method == "fp_v1_rescue_v2", descriptors, v)
            output, _ = self._stage(
                record, "exact",
                lambda: self._attention(q, k, tiles, indices, counts, scale, mean_desc, rescue,
                                        want_lse=False))
            if self.record:
                q_tile, k_tile = upstream.attention_tile_sizes()
                score_tile = upstream.score_tile_size() if self.method in V1_ROUTED_METHODS else None
                record["accounting"] = kernels.selection_accounting(
                    selected, q.shape[1], q_tile, k_tile, self.method, score_tile, self.block_size)

        if self.record and is_prefill:
            overall_end.record()
            record["events"]["attention"] = (overall_start, overall_end)
            self.profile_records.append(record)
        return output, None

    @staticmethod
    def _dense_accounting(query):
        sequence = query.shape[2]
        pairs = query.shape[0] * query.shape[1] * sequence * (sequence + 1) // 2
        return {
            "effective_exact_token_pair_ratio": 1.0,
            "exact_token_pairs": pairs,
            "causal_token_pairs": pairs,
            "legacy_block_density": 1.0,
            "selected_block_entries": None,
            "causal_block_entries": None,
            "exact_physical_qk_tiles": None,
            "mean_proxy_entries": 0,
            "selector_proxy_entries": 0,
            "mean_executed_logit_entries": 0,
            "mean_executed_value_entries": 0,
            "selector_executed_dot_entries": 0,
            "selector_physical_qk_tiles": None,
            "q_tile_size": None,
            "k_tile_size": None,
            "score_k_tile_size": None,
        }

    # ---------------------------------------------------- profile / capture

    def start_profile(self):
        self.profile_records.clear()
        self.record = True

    def start_capture(self, callback):
        """Attach a synchronous V1-prefill diagnostic callback."""
        self.capture_callback = callback

    def finish_capture(self):
        self.capture_callback = None

    def finish_profile(self):
        self.record = False
        torch.cuda.synchronize()
        rows = []
        for record in self.profile_records:
            row = {"layer": record["layer"], "method": record["method"]}
            for name in STAGE_NAMES:
                event = record["events"].get(name)
                row[f"{name}_ms"] = event[0].elapsed_time(event[1]) if event else 0.0
            for key, value in (record["accounting"] or {}).items():
                row[key] = value.item() if isinstance(value, torch.Tensor) else value
            rows.append(row)
        self.profile_records.clear()
        return rows
