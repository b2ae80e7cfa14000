"""Dense Q3.25 controller: drop-in for the reference's
mamba2_recall/state_quant_dense3.py (Dense3StateQuant, DenseStateQuant).

Same mixer orchestration as state_quant.StateQuant; the carry is the dense
3-bit codec (48 B of codes + 4 B of scales per row) driven by one table per
layer and group: a uint8 permutation or an int8 power-of-two equalizer.
"""
from __future__ import annotations

import torch

from . import state_codec_dense3 as dense3
from .state_quant import _MixerController

TABLE_KINDS = dense3.TABLE_KINDS


class Dense3StateQuant(_MixerController):
    """One [56,8,128] table, permutation or equalizer, never both
    (state_quant_dense3.py:10-27).  A batch-one cache including the
    convolution window is 28,499,968 bytes."""

    def __init__(self, model, table, *, table_kind="permutation"):
        if table_kind not in TABLE_KINDS:
            raise ValueError("Expected permutation or equalizer table")
        self.table_kind = table_kind
        super().__init__(model, "dense3_" + table_kind, table, False)

    def _validate_permutations(self, values):
        """state_quant_dense3.py:29-34."""
        if not isinstance(values, torch.Tensor) or tuple(values.shape) != self.TABLE_SHAPE:
            raise ValueError("Expected dense Q3 table[56,8,128]")
        cpu = values.detach().cpu().contiguous()
        layers, groups, n = self.TABLE_SHAPE
        dense3.validate_table(cpu.reshape(layers * groups, n), layers * groups, self.table_kind)
        return cpu.to(device=self.device).contiguous()

    @property
    def table(self):
        return self.permutations

    def _new_state(self, batch_size, index):
        return dense3.allocate_state(batch_size, self.HEADS, self.HEADDIM, self.D_STATE, self.device)

    def _scan_layer(self, index, mx, x, dt, aa, bm, cm, entry):
        y = dense3.scan(x, dt, aa, bm, cm, mx.D, mx.dt_bias, entry.state, self.permutations[index], self.table_kind)
        return y, None

    def assert_finite_cache(self):
        for entry in self._cache:
            dense3.validate_finite_result(entry.state)
        return True

    def cache_breakdown(self):
        """state_quant_dense3.py:108-125."""
        conv = sum(v.conv.numel() * v.conv.element_size() for v in self._cache)
        codes = sum(v.state.tensors["codes"].numel() for v in self._cache)
        scales = sum(v.state.tensors["scales"].numel() * 2 for v in self._cache)
        state = sum(v.state.nbytes for v in self._cache)
        if state != codes + scales:
            raise RuntimeError("Dense state storage differs from payload count")
        tables = self.permutations.numel() * self.permutations.element_size()
        return {"mode": self.mode, "table_kind": self.table_kind, "batch_size": self._batch_size,
                "allocated_layers": len(self._cache), "conv_fp16_bytes": conv, "ssm_payload_bytes": codes,
                "ssm_scale_bytes": scales, "ssm_total_bytes": state, "table_bytes": tables,
                "total_bytes": conv + state + tables, "calibration_workspace_bytes": 0,
                "tokens_per_layer": [v.tokens for v in self._cache],
                "scope": "Persistent request cache plus one compact table; weights, activations, registers, "
                         "allocator reserve and training workspace excluded"}


DenseStateQuant = Dense3StateQuant
