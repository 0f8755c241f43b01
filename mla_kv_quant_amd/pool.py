"""A packed-INT2 MLA cache pool carrying the attributes the reference writer reads.

The reference writer (deployment/sglang/QuantKernel/mla_fused_writer.py:110-224)
is handed SGLang's ``_PackedLatentMixin`` pool from an un-vendored fork. This
class holds the same attribute names and per-layer buffers, so the drop-in
entry points can be exercised without SGLang; a real SGLang pool with these
attributes works the same way.
"""

from __future__ import annotations

import torch

from .kernels import GROUP_SIZE


class PackedMLAPool:
    """Per-layer packed cache buffers (see ``include/rolaq_mla.h`` for layouts).

    ``rotations``: per-layer FP32 ``[D, D]`` rotations (or None); they are held
    in bf16, as the fork's pool holds them (``R_eff = fp32(bf16(R))``).
    ``quantizers``: per-layer ``(threshold, gain)`` or None (OSCAR default).
    """

    def __init__(self, size: int, layer_num: int, kv_lora_rank: int = 512, qk_rope_head_dim: int = 64,
                 max_reqs: int = 16, sink: int = 4, recent: int = 16, device="cuda",
                 rotations=None, quantizers=None, start_layer: int = 0, dtype=torch.bfloat16):
        if kv_lora_rank % GROUP_SIZE:
            raise ValueError("kv_lora_rank must be a multiple of 128")
        self.size = int(size)
        self.layer_num = int(layer_num)
        self.start_layer = int(start_layer)
        self.kv_lora_rank = int(kv_lora_rank)
        self.qk_rope_head_dim = int(qk_rope_head_dim)
        self.dtype = dtype
        self.device = torch.device(device)
        self._group_size = GROUP_SIZE
        self._bits = 2
        self._lloyd_max = True
        self._win_p = int(sink)
        self._win_r = int(recent)
        self._max_reqs = int(max_reqs)
        self._latent_windows = (sink + recent) > 0
        self._fb_window_meta: dict = {}
        self._selfcheck_budget = 0
        self._audit_budget = 0
        D, R, ng = self.kv_lora_rank, self.qk_rope_head_dim, self.kv_lora_rank // GROUP_SIZE
        slots = self.size + 1  # slot 0 is the graph-padding slot
        hp_rows = 1 + self._max_reqs * (self._win_p + self._win_r)
        dev = self.device
        self.c_codes = [torch.zeros(slots, D // 4, dtype=torch.uint8, device=dev) for _ in range(layer_num)]
        self.c_params = [torch.zeros(slots, ng, 2, dtype=torch.float32, device=dev) for _ in range(layer_num)]
        self.rope_buf = [torch.zeros(slots, R, dtype=dtype, device=dev) for _ in range(layer_num)]
        self.hp_c = [torch.zeros(hp_rows, D, dtype=dtype, device=dev) for _ in range(layer_num)]
        self.hp_row_of_slot = torch.full((slots,), -1, dtype=torch.int32, device=dev)
        self.hp_owner_of_row = torch.zeros(hp_rows, dtype=torch.int32, device=dev)
        rotations = rotations or [None] * layer_num
        self.rotations = [None if r is None else r.to(device=dev, dtype=dtype) for r in rotations]
        self._rolaq_quantizers = list(quantizers) if quantizers is not None else [None] * layer_num
        self._extend_ws = None  # the extend reader's key-row workspace, shared by all layers

    def extend_workspace(self, rows: int) -> torch.Tensor:
        """The extend reader's scratch of at least ``rows`` key rows (fp16
        ``[rows, D + R]``): one buffer for every layer and call, reallocated
        only when a batch needs more rows than it holds."""
        need = max(int(rows), 1)
        ws = self._extend_ws
        if ws is None or ws.shape[0] < need:
            ws = torch.empty(need, self.kv_lora_rank + self.qk_rope_head_dim, dtype=torch.float16,
                             device=self.device)
            self._extend_ws = ws
        return ws

    def latent_rotation(self, layer_id: int, local: bool = True):
        li = layer_id - self.start_layer if local else layer_id
        return self.rotations[li]

    def set_window_meta(self, is_decode: bool, seq_lens, req_pool_indices, fallback: bool = False):
        self._fb_window_meta = {"is_decode": is_decode, "seq_lens": seq_lens,
                                "req_pool_indices": req_pool_indices, "fallback": fallback}

    def get_kv_size_bytes(self) -> int:
        """Bytes of the packed cache: per-token rows of every layer plus the
        fixed BF16 window arena and the shared row map
        (rolaq_sglang.patch:166-189 charges the row map once, not per layer)."""
        D, R, ng = self.kv_lora_rank, self.qk_rope_head_dim, self.kv_lora_rank // GROUP_SIZE
        per_token = self.layer_num * (D // 4 + 8 * ng + 2 * R) + 4
        hp_rows = 1 + self._max_reqs * (self._win_p + self._win_r)
        return (self.size + 1) * per_token + hp_rows * (self.layer_num * D * 2 + 4)
