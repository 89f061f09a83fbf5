"""The forward's saved dict, with the reference's contract keys derived on demand.

``FusedMoEForward.forward(..., return_saved=True)`` stores what the backward
here reads (routing tables, references to the inputs, the saved FC1 output).
The reference's native saved dict (``ops/_native_saved.py:127-246``,
``ops/_single_saved_adapter.py:64-68``) carries more keys: zero-copy weight
views, plan metadata clones, grouped-GEMM tile tables, the send / receive
permutation pairs and host-side counts. On one GPU every one of them is a
closed form of the tables already saved, so ``MoESaved`` computes a key the
first time it is read and keeps it. The backward never reads them, so the
forward → backward path pays nothing for them and makes no host read (it
stays capturable in a HIP graph); a caller that inspects, say, ``total_recv``
triggers one device-to-host read, as the reference's snapshot does.

World size 1 fixes the transport-side tables: the single source rank's
arrival order is the expert-major slot order (``local_sort_idxs`` is the
identity), send buckets coincide with the expert offsets, and the
per-(rank, expert) count matrices are ``[1, E]`` views of the counts.
"""

from __future__ import annotations

import torch

# Row tile of the reference's grouped-GEMM metadata (ops/_torch_forward.py:28).
META_BLOCK_SIZE_M = 64


class MoESaved(dict):
    """dict of the saved activations and tables; reference contract keys are
    derived on first access (``saved[key]``, ``saved.get(key)``, ``key in saved``)."""

    _DERIVED = (
        # zero-copy weight views (_native_saved.py:384-401) and input references
        "fc1_combined", "fc1_1", "fc1_2",
        # minimal single-kernel contract (_single_saved_adapter.py:64-68)
        "recv_expert_offsets", "recv_counts_by_source_expert", "forward_send_route",
        # plan metadata (_native_saved.py:127-233)
        "num_tiles_total", "meta_expert_ids", "meta_split_cum", "meta_tile_num", "meta_tile_num_cum",
        "plan_send_counts_by_rank_expert", "plan_send_bucket_starts", "plan_send_bucket_dst_starts",
        "plan_recv_counts_by_source_expert", "plan_received_expert_offsets",
        # permutation pairs
        "sort_idxs", "inv_sort", "local_sort_idxs", "inv_local",
        # host values
        "total_send", "total_recv", "M", "splits_send_list", "splits_recv_list",
        # the dispatched-token copy (a gather, materialised only when read)
        "recv_hidden_sorted",
    )

    def __missing__(self, key):
        if key not in self._DERIVED:
            raise KeyError(key)
        value = self._derive(key)
        self[key] = value
        return value

    def __contains__(self, key):
        return dict.__contains__(self, key) or (key in self._DERIVED and self._has_tables())

    def get(self, key, default=None):
        try:
            return self[key]
        except KeyError:
            return default

    def _has_tables(self) -> bool:
        return dict.__contains__(self, "split_size_cum_per_expert")

    # ------------------------------------------------------------ derivations
    def _num_valid(self) -> int:
        if not dict.__contains__(self, "_num_valid"):
            offsets = dict.__getitem__(self, "split_size_cum_per_expert")
            dict.__setitem__(self, "_num_valid", int(offsets[-1].item()))
        return dict.__getitem__(self, "_num_valid")

    def _derive(self, key):
        if not self._has_tables():
            raise KeyError(key)
        g = lambda k: dict.__getitem__(self, k)  # noqa: E731 (stored keys only)
        E = g("experts_per_rank")
        F = g("ffn_dim")
        offsets = g("split_size_cum_per_expert")
        counts = g("expert_counts")
        device = offsets.device
        if key in ("fc1_combined", "fc1_1", "fc1_2"):
            w1 = g("gate_up_weight")
            return {"fc1_combined": w1.transpose(1, 2), "fc1_1": w1[:, :, :F].transpose(1, 2),
                    "fc1_2": w1[:, :, F:].transpose(1, 2)}[key]
        if key in ("recv_expert_offsets", "plan_received_expert_offsets"):
            return offsets
        if key in ("recv_counts_by_source_expert", "plan_recv_counts_by_source_expert",
                   "plan_send_counts_by_rank_expert"):
            return counts.view(1, E)
        if key in ("plan_send_bucket_starts", "plan_send_bucket_dst_starts"):
            return offsets[:E]
        if key in ("total_send", "total_recv", "M"):
            return self._num_valid()
        if key in ("splits_send_list", "splits_recv_list"):
            return [self._num_valid()]
        n = self._num_valid()
        if key == "forward_send_route":
            return g("send_route_indices")[:n].contiguous()
        if key == "sort_idxs":
            return g("send_route_indices")[:n].to(torch.int64)
        if key == "inv_sort":
            # argsort of the send order (_native_saved.py:220); its values are
            # distinct route ids, so this is the inverse permutation when no
            # route is dropped
            return torch.argsort(self["sort_idxs"], stable=True)
        if key in ("local_sort_idxs", "inv_local"):
            return torch.arange(n, dtype=torch.int64, device=device)
        if key == "recv_hidden_sorted":
            return g("hidden_states").index_select(0, g("send_token_indices")[:n].to(torch.int64))
        # grouped-GEMM tile tables (_native_saved.py:146-188)
        c64 = counts.to(torch.int64)
        tiles = (c64 + META_BLOCK_SIZE_M - 1) // META_BLOCK_SIZE_M
        num_tiles = int(tiles.sum().item())
        if key == "num_tiles_total":
            return torch.tensor([num_tiles], dtype=torch.int32, device=device)
        if num_tiles == 0:
            return torch.empty(0, dtype=torch.int32, device=device)
        token_starts = c64.cumsum(0) - c64
        tile_starts = tiles.cumsum(0) - tiles
        if key == "meta_expert_ids":
            v = torch.repeat_interleave(torch.arange(E, dtype=torch.int64, device=device), tiles,
                                        output_size=num_tiles)
        elif key == "meta_split_cum":
            v = torch.repeat_interleave(token_starts, tiles, output_size=num_tiles)
        elif key == "meta_tile_num_cum":
            v = torch.repeat_interleave(tile_starts, tiles, output_size=num_tiles)
        else:  # meta_tile_num
            v = (torch.arange(num_tiles, dtype=torch.int64, device=device)
                 - torch.repeat_interleave(tile_starts, tiles, output_size=num_tiles))
        return v.to(torch.int32)
