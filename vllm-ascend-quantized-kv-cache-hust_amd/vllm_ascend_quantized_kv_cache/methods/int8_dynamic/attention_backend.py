# SPDX-License-Identifier: Apache-2.0
"""INT8 dynamic per-channel attention mixin.

Role of ``AscendInt8AttentionBackendMixin`` in the reference
(``pkg/methods/int8_dynamic/attention_backend.py``, cited as ``i8ab.py``):
scales are computed once per layer from the first K/V it sees, every step
quantizes and writes the int8 pages, and the attention state picks decode,
chunked prefill or prefill.  Here the quantize and the page write are one
HIP kernel (the reference quantizes in torch and hands the codes to the
host's ``reshape_and_cache``), decode is a fused HIP kernel with per-channel
antiquant, and prefill over cached pages dequantizes to dense TND and runs
the MFMA attention kernel.  Pooling encoders stay with the host and are
refused here.  Under graph capture the reference hands the decode to the
host's ``full_graph_fia`` (``i8ab.py:97-104``); here a captured ``forward``
records the layer's capturable decode step (``int8_decode_graph``), whose
plan the host stages before every replay (``prepare_int8_graph_replay``),
and refuses every other capture.
"""

from __future__ import annotations

from typing import Any

import numpy as np
import torch

from ...core.runtime import stream_capturing


def _state(attn_metadata: Any) -> str:
    state = getattr(attn_metadata, "attn_state", None)
    if state is None:
        return "UNKNOWN"
    return getattr(state, "name", None) or str(state)


class AscendInt8AttentionBackendMixin:
    """Runtime-calibrated INT8 KV cache on the MI355X kernels."""

    key_cache: Any = None
    value_cache: Any = None
    #: capturable decode steps by batch size (``int8_decode_graph``)
    _int8_capture_graphs: dict | None = None

    def forward(
        self,
        layer: Any,
        query: torch.Tensor,
        key: torch.Tensor,
        value: torch.Tensor,
        kv_cache: Any,
        attn_metadata: Any,
        output: torch.Tensor | None = None,
        output_scale: torch.Tensor | None = None,
        output_block_scale: torch.Tensor | None = None,
    ) -> torch.Tensor:
        """INT8 forward entry (``i8ab.py:34-128``)."""
        assert output is not None, "Output tensor must be provided."
        if output_scale is not None or output_block_scale is not None:
            raise NotImplementedError(
                "fused output quantization is not yet supported for "
                "AscendInt8AttentionBackendImpl"
            )
        assert getattr(layer, "_k_scale_float", 1.0) == 1.0
        assert getattr(layer, "_v_scale_float", 1.0) == 1.0
        if attn_metadata is None:
            return output.fill_(0)
        if stream_capturing():
            return self._forward_int8_captured(query, key, value, attn_metadata, output)

        if self.key_cache is None and kv_cache is not None:
            if (isinstance(kv_cache, torch.Tensor) and kv_cache.dim() > 0
                    and kv_cache.shape[0] == 2) or (
                    isinstance(kv_cache, list | tuple) and len(kv_cache) >= 2):
                self.key_cache, self.value_cache = kv_cache[0], kv_cache[1]

        state = _state(attn_metadata)
        float_key = float_value = None
        step = False
        if key is not None and value is not None:
            if state != "DecodeOnly":
                float_key, float_value = key, value
            self._prepare_int8_scales(layer, key, value)
            n = min(int(getattr(attn_metadata, "num_actual_tokens", key.shape[0])), key.shape[0])
            # a decode step of one token per request writes its tokens inside
            # the planned step (slots from the staged plan)
            step = (state == "DecodeOnly" and self._int8_step_enabled(query)
                    and n == len(attn_metadata.seq_lens_list))
            if not step:
                self._write_int8_cache(key[:n], value[:n], attn_metadata.slot_mapping[:n], layer)
        elif state == "DecodeOnly" and getattr(layer, "_int8_scales_ready", False):
            step = self._int8_step_enabled(query)

        if getattr(attn_metadata, "model_runner_type", None) == "pooling" and not getattr(
            attn_metadata, "causal", True
        ):
            raise NotImplementedError(
                "encoder-only (pooling) attention stays on the host attention backend"
            )
        if not getattr(layer, "_int8_scales_ready", False):
            raise RuntimeError(
                "INT8 KV cache has no scales yet: the first forward of a layer must "
                "carry key/value to calibrate them."
            )
        if state == "DecodeOnly":
            if step:
                return self._forward_int8_decode_step(query, key, value, attn_metadata, output,
                                                      layer)
            return self._forward_int8_decode(query, attn_metadata, output, layer)
        if state == "ChunkedPrefill":
            return self._forward_int8_chunked_prefill(
                query, float_key, float_value, attn_metadata, output, layer
            )
        return self._forward_int8_prefill(
            query, float_key, float_value, attn_metadata, output, layer
        )

    def _forward_int8_captured(self, query: Any, key: Any, value: Any, attn_metadata: Any,
                               output: Any) -> Any:
        """``forward`` while the host records a HIP graph (``i8ab.py:97-104``).

        The eager decode stages a one-step plan (slots, lengths, the split-K
        work list) from host memory, and a recorded copy of it would replay
        that one step forever.  Only the decode step of a batch whose
        capturable form the host created beforehand (``int8_decode_graph``) is
        recorded: its launches read a persistent plan buffer that
        ``prepare_int8_graph_replay`` refills before each replay.  Prefill,
        chunked prefill and uncalibrated layers are refused.
        """
        b = len(attn_metadata.seq_lens_list)
        graph = self._int8_capture_graphs.get(b) if self._int8_capture_graphs else None
        if _state(attn_metadata) != "DecodeOnly" or graph is None:
            raise RuntimeError(
                "INT8 forward() was called under HIP graph capture: its eager step stages a "
                "one-step plan that every replay would reuse. Capture only decode steps, after "
                f"creating the batch-{b} capturable step with "
                "impl.int8_decode_graph(layer, batch, max_blocks=...), and call "
                "impl.prepare_int8_graph_replay(attn_metadata) before every replay; or run the "
                "layer eagerly."
            )
        return graph.launch(query, key, value, output)

    def prepare_int8_graph_replay(self, attn_metadata: Any) -> None:
        """Stage the plan of the step a captured ``forward`` will replay next
        (the batch's ``Int8DecodeGraph.prepare``)."""
        b = len(attn_metadata.seq_lens_list)
        graph = self._int8_capture_graphs.get(b) if self._int8_capture_graphs else None
        if graph is None:
            raise RuntimeError(f"INT8 decode graph: no capturable step for batch {b}.")
        graph.prepare(attn_metadata)

    # -- scales and quantize (i8ab.py:130-171) ------------------------------

    def _prepare_int8_scales(self, layer: Any, key: torch.Tensor, value: torch.Tensor) -> None:
        """Scales from the whole first K/V (padding rows included, i8ab.py:82)."""
        if getattr(layer, "_int8_scales_ready", False):
            return
        from ...ops.int8_ops import int8_calc_scales

        k_inv, v_inv, k_aq, v_aq = int8_calc_scales(key, value)
        layer._int8_k_inv_scale = k_inv
        layer._int8_v_inv_scale = v_inv
        layer._int8_k_offset = torch.zeros_like(k_inv)
        layer._int8_v_offset = torch.zeros_like(v_inv)
        layer._int8_k_aq_scale = k_aq
        layer._int8_v_aq_scale = v_aq
        layer._int8_k_aq_offset = torch.zeros_like(k_aq)
        layer._int8_v_aq_offset = torch.zeros_like(v_aq)
        layer._int8_scales_ready = True

    @staticmethod
    def _quantize_kv_to_runtime_int8(
        key: torch.Tensor, value: torch.Tensor, layer: Any, num_actual_tokens: int
    ) -> tuple[torch.Tensor, torch.Tensor]:
        from ...ops.int8_ops import int8_quantize

        return (
            int8_quantize(key[:num_actual_tokens], layer._int8_k_inv_scale),
            int8_quantize(value[:num_actual_tokens], layer._int8_v_inv_scale),
        )

    def _write_int8_cache(self, key: Any, value: Any, slot_mapping: Any, layer: Any) -> None:
        """Quantize and write the step's K/V into the int8 pages (one kernel)."""
        if self.key_cache is None:
            raise RuntimeError("INT8 KV cache tensors are not bound.")
        from ...ops.int8_ops import int8_quant_scatter

        int8_quant_scatter(key, value, layer._int8_k_inv_scale, layer._int8_v_inv_scale,
                           slot_mapping, self.key_cache, self.value_cache)

    # -- attention (i8ab.py:173-404) ---------------------------------------

    def _forward_int8_decode(self, query: Any, attn_metadata: Any, output: Any, layer: Any) -> Any:
        from ...ops.int8_ops import int8_decode_attention

        seq_lens = [int(x) for x in attn_metadata.seq_lens_list]
        b = len(seq_lens)
        out = output[:b].view(b, self.num_heads, self.head_size)
        got = int8_decode_attention(
            query[:b].reshape(b, self.num_heads, self.head_size).contiguous(),
            self.key_cache, self.value_cache, layer._int8_k_aq_scale, layer._int8_v_aq_scale,
            attn_metadata.block_tables[:b], seq_lens, self.scale, out=out,
        )
        if got is not out:
            out.copy_(got)
        return output

    # -- decode step from a host plan (sync-free, capturable launches) -----

    def _int8_step_enabled(self, query: Any) -> bool:
        """The planned INT8 step applies: the step's tensors are on the GPU."""
        return isinstance(query, torch.Tensor) and query.device.type == "cuda" and (
            self.key_cache is not None and self.key_cache.device.type == "cuda")

    def _int8_host_slots(self, attn_metadata: Any, n: int) -> np.ndarray:
        """The step's slots as host int64, from the host's copy when present."""
        host = getattr(attn_metadata, "slot_mapping_cpu", None)
        x = host if host is not None else attn_metadata.slot_mapping
        if isinstance(x, torch.Tensor):
            if x.device.type != "cpu":
                self.int8_host_reads = getattr(self, "int8_host_reads", 0) + 1
                x = x.cpu()
            x = x.numpy()
        return np.asarray(x[:n], dtype=np.int64)

    def _forward_int8_decode_step(self, query: Any, key: Any, value: Any, attn_metadata: Any,
                                  output: Any, layer: Any) -> Any:
        """Quantize + scatter, fused decode and combine over one staged plan."""
        from ...ops.int8_ops import int8_split_tokens
        from .decode_step import Int8StepBuffers, launch_int8_step

        lens = [int(x) for x in attn_metadata.seq_lens_list]
        b = len(lens)
        if b == 0:
            return output
        bs = self.key_cache.shape[1]
        table = attn_metadata.block_tables[:b]
        if max(lens) > table.shape[1] * bs or min(lens) < 0:
            raise ValueError(
                f"int8_decode_attention: a sequence length exceeds its block table "
                f"({max(lens)} > {table.shape[1]} x {bs})"
            )
        split = int8_split_tokens(sum(lens), self.num_kv_heads, seq_lens=lens)
        need = b + sum(-(-n // split) for n in lens)
        bufs = getattr(self, "_int8_step_bufs", None)
        if bufs is None or bufs.batch < b or bufs.work_cap < need:
            bufs = Int8StepBuffers(query.device, batch=max(b, 2 * (bufs.batch if bufs else 0)),
                                   work_cap=2 * need, num_heads=self.num_heads,
                                   head_size=self.head_size)
            self._int8_step_bufs = bufs
        slots = None if key is None else self._int8_host_slots(attn_metadata, b)
        count = bufs.stage(slots, lens, split, fixed=False)
        kvh, d = self.num_kv_heads, self.head_size
        k = None if key is None else key[:b].reshape(b, kvh, d).contiguous()
        v = None if value is None else value[:b].reshape(b, kvh, d).to(k.dtype).contiguous()
        out = output[:b].view(b, self.num_heads, d)
        launch_int8_step(self, bufs, layer, query[:b].reshape(b, self.num_heads, d).contiguous(),
                         k, v, table.to(torch.int32).contiguous(), count, out)
        return output

    def int8_decode_graph(self, layer: Any, batch: int, *, max_blocks: int):
        """An ``Int8DecodeGraph`` for this layer (calibrated scales, bound
        cache): the decode step's launches, capturable once in a HIP graph
        and replayed every step after ``prepare`` stages that step's plan."""
        from .decode_step import Int8DecodeGraph

        graph = Int8DecodeGraph(self, layer, batch, max_blocks=max_blocks)
        if self._int8_capture_graphs is None:
            self._int8_capture_graphs = {}
        self._int8_capture_graphs[batch] = graph  # what a captured forward() launches
        return graph

    def _dense_attention(self, q: Any, k: Any, v: Any, q_lens: list[int], kv_lens: list[int],
                         causal: bool, out: Any) -> Any:
        from ...ops.attention import prefill_attention

        return prefill_attention(q, k, v, q_lens, kv_lens, self.scale, causal, out=out)

    def _forward_int8_chunked_prefill(self, query: Any, float_key: Any, float_value: Any,
                                      attn_metadata: Any, output: Any, layer: Any) -> Any:
        nd = attn_metadata.num_decode_tokens
        ndr = attn_metadata.num_decodes
        qlen = [int(x) for x in attn_metadata.actual_seq_lengths_q]
        num_tokens = qlen[-1]
        seq_lens = [int(x) for x in attn_metadata.seq_lens_list]
        if nd > 0:
            from ...ops.int8_ops import int8_decode_attention

            out = output[:nd].view(nd, self.num_heads, self.head_size)
            got = int8_decode_attention(
                query[:nd].reshape(nd, self.num_heads, self.head_size).contiguous(),
                self.key_cache, self.value_cache, layer._int8_k_aq_scale,
                layer._int8_v_aq_scale, attn_metadata.block_tables[:ndr], seq_lens[:ndr],
                self.scale, out=out,
            )
            if got is not out:
                out.copy_(got)
        if attn_metadata.num_prefills > 0:
            q_lens = [qlen[i] - (qlen[i - 1] if i > 0 else 0) for i in range(ndr, len(qlen))]
            all_new = all(seq_lens[i] <= q_lens[i - ndr] for i in range(ndr, len(seq_lens)))
            if all_new and float_key is not None and float_value is not None:
                k = float_key[nd:num_tokens]
                v = float_value[nd:num_tokens]
                kv_lens = q_lens
            else:
                k, v = self._dequant_int8_paged_kv_to_dense(
                    self.key_cache, self.value_cache, attn_metadata.block_tables[ndr:],
                    seq_lens[ndr:], query.dtype, layer,
                )
                kv_lens = seq_lens[ndr:]
            n = num_tokens - nd
            out = output[nd:num_tokens].view(n, self.num_heads, self.head_size)
            self._dense_attention(
                query[nd:num_tokens].reshape(n, self.num_heads, self.head_size), k, v, q_lens,
                kv_lens, True, out,
            )
        return output

    def _forward_int8_prefill(self, query: Any, float_key: Any, float_value: Any,
                              attn_metadata: Any, output: Any, layer: Any) -> Any:
        qlen = [int(x) for x in attn_metadata.actual_seq_lengths_q]
        num_tokens = qlen[-1]
        q_lens = [qlen[i] - (qlen[i - 1] if i > 0 else 0) for i in range(len(qlen))]
        seq_lens = [int(x) for x in getattr(attn_metadata, "seq_lens_list", q_lens)]
        if _state(attn_metadata) == "PrefillNoCache" and float_key is not None:
            k, v, kv_lens = float_key[:num_tokens], float_value[:num_tokens], q_lens
        else:
            k, v = self._dequant_int8_paged_kv_to_dense(
                self.key_cache, self.value_cache, attn_metadata.block_tables, seq_lens,
                query.dtype, layer,
            )
            kv_lens = seq_lens
        out = output[:num_tokens].view(num_tokens, self.num_heads, self.head_size)
        self._dense_attention(
            query[:num_tokens].reshape(num_tokens, self.num_heads, self.head_size), k, v,
            q_lens, kv_lens, True, out,
        )
        return output

    def _dequant_int8_paged_kv_to_dense(self, key: Any, value: Any, block_table: Any,
                                        seq_lens: list[int], target_dtype: Any,
                                        layer: Any) -> tuple[Any, Any]:
        from ...ops.int8_ops import int8_dequant_gather

        nb = key.shape[0]
        bs = key.shape[1]
        kc = key.view(nb, bs, self.num_kv_heads, self.head_size)
        vc = value.view(nb, bs, self.num_kv_heads, self.head_size)
        aq_k = (1.0 / layer._int8_k_inv_scale.to(target_dtype))
        aq_v = (1.0 / layer._int8_v_inv_scale.to(target_dtype))
        return int8_dequant_gather(kc, vc, block_table[: len(seq_lens)], seq_lens, target_dtype,
                                   aq_k, aq_v)


__all__ = ["AscendInt8AttentionBackendMixin"]
