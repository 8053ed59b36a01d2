"""Packed variable-length sequences (``cu_seqlens``) for the ops and the retriever.

Convention of the FLA kernels the reference vendors (gated_delta_rule/
fused_recurrent.py:379-437) and of the flash_moba varlen calls it makes
(modelings/modeling_sgsa.py:231-300): the sequences are packed along the token
dimension of a batch of one, ``x [1, total, ...]``, and ``cu_seqlens [N+1]``
(int32 or int64, cu_seqlens[0] == 0, non-decreasing, cu_seqlens[N] == total)
bounds sequence n to tokens [cu_seqlens[n], cu_seqlens[n+1]).  Initial and
final states are per sequence, [N, H, D, D].

The sequences are laid out as the rows of a padded batch [N, L_max] (one copy
in each direction, a row gather on the GPU) and run through the masked kernels
or, for the chunked state update, with pads that leave the state unchanged
(beta = alpha = 0, gamma = 1).  Every sequence starts at position 0 of its own
row, so causality, block boundaries (multiples of block_size from the
sequence start) and retrieved indices are relative to the sequence start, as
in the varlen kernels.  The layout copies are differentiable.
"""

from __future__ import annotations

from typing import Optional, Sequence

import torch
from torch import Tensor


class SeqLayout:
    """Where each packed token sits in the padded batch [N, L_max]."""

    def __init__(self, cu_seqlens: Tensor, total: int, device: torch.device) -> None:
        if cu_seqlens.dim() != 1 or cu_seqlens.numel() < 2:
            raise ValueError("cu_seqlens must be a 1-D tensor of N+1 >= 2 offsets")
        if cu_seqlens.dtype not in (torch.int32, torch.int64):
            raise ValueError(f"cu_seqlens must be int32 or int64, got {cu_seqlens.dtype}")
        cu = cu_seqlens.detach().to("cpu", torch.int64)
        lens = cu[1:] - cu[:-1]
        if int(cu[0]) != 0 or bool((lens < 0).any()) or int(cu[-1]) != total:
            raise ValueError(f"cu_seqlens must start at 0, not decrease and end at the {total} packed tokens; "
                             f"got {cu.tolist()}")
        self.n = int(lens.numel())
        self.max_len = max(int(lens.max()), 1)
        self.total = total
        self.lengths = lens
        seq = torch.repeat_interleave(torch.arange(self.n), lens)
        pos = torch.arange(total) - cu[:-1][seq]
        self.flat = (seq * self.max_len + pos).to(device)     # packed token -> padded row index
        pad_mask = torch.zeros(self.n * self.max_len, dtype=torch.bool)
        pad_mask[seq * self.max_len + pos] = True
        self.mask = pad_mask.view(self.n, self.max_len).to(device)   # [N, L_max], True = real token

    def pad(self, x: Tensor, fill: float = 0.0) -> Tensor:
        """x [1, total, *rest] -> [N, L_max, *rest], ``fill`` in the pads."""
        if x.shape[0] != 1 or x.shape[1] != self.total:
            raise ValueError(f"packed inputs must be [1, {self.total}, ...], got {tuple(x.shape)}")
        rest = tuple(x.shape[2:])
        out = x.new_full((self.n * self.max_len,) + rest, fill)
        return out.index_copy(0, self.flat, x[0]).view((self.n, self.max_len) + rest)

    def unpad(self, y: Tensor) -> Tensor:
        """y [N, L_max, *rest] -> [1, total, *rest]."""
        rest = tuple(y.shape[2:])
        return y.reshape((self.n * self.max_len,) + rest).index_select(0, self.flat).unsqueeze(0)

    def unpad_rows(self, y: Tensor) -> Tensor:
        """Per-row outputs [N, H, L_max, *rest] -> [1, H, total, *rest]."""
        return self.unpad(y.transpose(1, 2)).transpose(1, 2)


def layout(cu_seqlens: Tensor, x: Tensor) -> SeqLayout:
    """The layout of packed ``x [1, total, ...]`` under ``cu_seqlens``."""
    if x.dim() < 2 or x.shape[0] != 1:
        raise ValueError(f"with cu_seqlens the batch size must be 1 (sequences packed along dim 1), "
                         f"got {tuple(x.shape)}")
    return SeqLayout(cu_seqlens, x.shape[1], x.device)


def check_states(lay: SeqLayout, initial_state: Optional[Tensor]) -> None:
    if initial_state is not None and initial_state.shape[0] != lay.n:
        raise ValueError(f"with cu_seqlens the initial state holds one state per sequence: "
                         f"[{lay.n}, H, D, D], got {tuple(initial_state.shape)}")


def pad_state_inputs(lay: SeqLayout, q: Tensor, k: Tensor, v: Tensor, beta: Tensor, gamma: Tensor,
                     sparse_k: Optional[Tensor], sparse_v: Optional[Tensor],
                     alpha: Optional[Tensor]) -> Sequence[Optional[Tensor]]:
    """The state-update inputs on the padded batch; pads write nothing (beta =
    alpha = 0) and do not decay the state (gamma = 1), so each row's final state
    is its sequence's."""
    p = lay.pad
    return (p(q), p(k), p(v), p(beta), p(gamma, 1.0),
            p(sparse_k) if sparse_k is not None else None,
            p(sparse_v) if sparse_v is not None else None,
            p(alpha) if alpha is not None else None)


# retrieval outputs laid out per token, [B,T,H,*]; every other tensor output is per row, [B,H,T,*]
_TOKEN_MAJOR = ("k_hat", "v_hat")


def unpad_retrieval(lay: SeqLayout, r: dict) -> dict:
    """A retrieval dict of the padded batch back to the packed layout: k_hat /
    v_hat [1,total,H,D]; indices, weights, scores, counts, validity, block
    indices / scores and each diagnostic [1,H,total,*].  Indices stay relative to
    the start of their sequence."""
    out = {}
    for name, val in r.items():
        if isinstance(val, dict):
            out[name] = {n: lay.unpad_rows(t) for n, t in val.items()}
        elif isinstance(val, Tensor):
            out[name] = lay.unpad(val) if name in _TOKEN_MAJOR else lay.unpad_rows(val)
        else:
            out[name] = val
    return out
