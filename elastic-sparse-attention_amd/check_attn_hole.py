"""Attention-hole checker on the GPU.

Drop-in for the reference's ``check_attn_hole.py``
(HighCWu/elastic-sparse-attention): ``check_attention_holes_pytorch``
(:53-180) asks whether one position can see its whole history through the
stacked elastic layers.  The last layer gives the position's own valid
indices over all heads (:102-116); every earlier layer adds the valid
indices of every token reached so far (:134-159); a token never reached is a
hole.

The reference materialises each layer's ``[H, L, w]`` int64 index set on the
device and grows a boolean set with gathers and ``unique()``.  Here one C-ABI
call (``esa_reachability``) runs the whole propagation as bitmap passes that
regenerate the indices in-kernel (bit-exact with the layout builder), so the
memory is two bitmaps of ``L / 8`` bytes.  ``attention_reachability`` returns
the result; ``check_attention_holes_pytorch`` prints the reference's report.
"""
from __future__ import annotations

import ctypes
import time
from dataclasses import dataclass
from typing import List, Optional

import torch

from esa_native import check, load

__all__ = ["Reachability", "attention_reachability", "check_attention_holes_pytorch"]


@dataclass
class Reachability:
    """Receptive field of ``position``: ``reachable`` is bool ``[position + 1]``
    on the device; ``layer_counts`` the set size after each layer, last layer
    first."""
    position: int
    reachable: torch.Tensor
    layer_counts: List[int]

    @property
    def num_reachable(self) -> int:
        return self.layer_counts[-1] if self.layer_counts else int(self.reachable.sum())

    @property
    def holes(self) -> int:
        return self.position + 1 - self.num_reachable

    def unreachable(self) -> torch.Tensor:
        """Indices of the tokens the position cannot see, ascending."""
        return torch.where(~self.reachable)[0]


def _stream(device: torch.device) -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def attention_reachability(seq_len: int, num_hidden_layers: int, num_attention_heads: int,
                           attn_length: int, position_id: Optional[int] = None,
                           device: Optional[torch.device] = None) -> Reachability:
    """Tokens ``position_id`` (default ``seq_len - 1``) reaches through
    ``num_hidden_layers`` elastic layers of ``num_attention_heads`` heads and
    window ``attn_length`` (check_attn_hole.py:53-163).  Raises ``ValueError``
    for a position outside ``[0, seq_len)`` (:75-76) or a non-positive
    ``attn_length``."""
    if position_id is None:
        target = seq_len - 1
    else:
        if not (0 <= position_id < seq_len):
            raise ValueError(
                f"position_id must be between 0 and {seq_len - 1}, but got {position_id}")
        target = position_id
    if attn_length <= 0:
        raise ValueError("attn_length must be positive.")
    dev = torch.device("cuda", torch.cuda.current_device()) if device is None else torch.device(device)
    if dev.type != "cuda":
        raise RuntimeError("attention_reachability runs on the GPU; got device " + str(dev))
    n = target + 1
    nwords = (n + 31) // 32
    reach = torch.empty(nwords, dtype=torch.int32, device=dev)
    work = torch.empty(nwords, dtype=torch.int32, device=dev)
    counts = torch.empty(max(num_hidden_layers, 1), dtype=torch.int32, device=dev)
    check(load().esa_reachability(seq_len, attn_length, num_hidden_layers, num_attention_heads,
                                  target, ctypes.c_void_p(reach.data_ptr()),
                                  ctypes.c_void_p(work.data_ptr()),
                                  ctypes.c_void_p(counts.data_ptr()), _stream(dev)),
          "esa_reachability")
    shifts = torch.arange(32, dtype=torch.int32, device=dev)
    bits = ((reach.view(-1, 1) >> shifts) & 1).view(-1)[:n].bool()
    return Reachability(target, bits, [int(c) for c in counts[:num_hidden_layers].cpu()])


def check_attention_holes_pytorch(seq_len: int, num_hidden_layers: int, num_attention_heads: int,
                                  attn_length: int, position_id: Optional[int] = None
                                  ) -> Optional[Reachability]:
    """Prints the reference's report (check_attn_hole.py:53-180) for one
    position and returns the ``Reachability`` (the reference returns
    nothing).  Without a GPU it prints a notice and returns ``None``, as the
    reference does (:66-68)."""
    if not torch.cuda.is_available():
        print("No GPU is available. Skipping this test.")
        return None
    target = seq_len - 1 if position_id is None else position_id
    if position_id is not None and not (0 <= position_id < seq_len):
        raise ValueError(
            f"position_id must be between 0 and {seq_len - 1}, but got {position_id}")
    print(f"\n--- Checking with attn_length = {attn_length}, seq_len = {seq_len} ---")
    print(f"--- Target position to check: {target} ---")
    if attn_length <= 0:
        print("Error: attn_length must be positive.")
        return None
    start = time.time()
    r = attention_reachability(seq_len, num_hidden_layers, num_attention_heads, attn_length,
                               target)
    elapsed = time.time() - start
    history_len = target + 1
    for k, count in enumerate(r.layer_counts):
        print(f"[{elapsed:.2f}s] After layer {num_hidden_layers - 1 - k}, pos {target} "
              f"can see {count} tokens.")
        # the reference tests for a full set after each earlier layer (:161-163)
        if k > 0 and count == history_len:
            print(f"[{elapsed:.2f}s] Full history reachability achieved. Stopping.")
            break
    print(f"\n--- Test complete in {elapsed:.2f} seconds ---")
    if r.holes == 0:
        print(f"SUCCESS: Position {target} has no attention holes. It can see all "
              f"{history_len} previous tokens (including itself).")
    else:
        print(f"FAILURE: Position {target} has {r.holes} attention holes in its history.")
        print("   It CANNOT see its complete history.")
        print(f"   Example unreachable indices: {r.unreachable()[:10].tolist()}")
    return r


if __name__ == "__main__":
    # the reference script's three checks (check_attn_hole.py:182-234)
    check_attention_holes_pytorch(seq_len=131072, num_hidden_layers=8, num_attention_heads=8,
                                  attn_length=64, position_id=131071)
    check_attention_holes_pytorch(seq_len=131072, num_hidden_layers=8, num_attention_heads=8,
                                  attn_length=64, position_id=4095)
    check_attention_holes_pytorch(seq_len=131072, num_hidden_layers=8, num_attention_heads=8,
                                  attn_length=16, position_id=32767)
