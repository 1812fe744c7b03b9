"""Shared module-substitution walk of quantize_module_int4 / _fp8.

The reference's plugin API is attribute substitution: a bias-free
``nn.Linear`` child whose attribute name is a target and whose weight is at
least ``min_bytes`` is replaced in its parent by a quantized module
(models/int4_linear.py:137-153, models/fp8_linear.py:104-114).  The stats the
callers report (converted / below threshold / unsupported / bytes saved) are
part of that API, so the walk keeps the reference's counting rules:
  * children that are not bias-free Linears, or whose name is not a target,
    are not counted at all;
  * a small target counts as below threshold;
  * a target whose replacement raises counts as unsupported when the caller
    tolerates construction errors, and the original is kept.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Callable, Iterable

from torch import nn


@dataclass
class SwapStats:
    converted: int = 0
    small: int = 0
    unsupported: int = 0
    saved: int = 0


def _candidates(root: nn.Module, target_names: Iterable[str]):
    """(parent, attribute, linear) for every bias-free Linear child whose
    attribute name is a target (all names when target_names is empty)."""
    targets = set(target_names or ())
    found = []
    for parent in root.modules():
        for attr, child in parent.named_children():
            if not isinstance(child, nn.Linear) or child.bias is not None:
                continue
            if targets and attr not in targets:
                continue
            found.append((parent, attr, child))
    return found


def swap_linears(
    root: nn.Module,
    target_names: Iterable[str],
    min_bytes: int,
    build: Callable[[nn.Linear], nn.Module],
    saved_bytes: Callable[[int], int],
    tolerate_errors: bool,
    drop_original: bool,
) -> SwapStats:
    stats = SwapStats()
    # Collect first, then substitute: replacements are never revisited.
    for parent, attr, linear in _candidates(root, target_names):
        nbytes = linear.weight.numel() * linear.weight.element_size()
        if nbytes < min_bytes:
            stats.small += 1
            continue
        if tolerate_errors:
            try:
                new = build(linear)
            except Exception:  # noqa: BLE001 - geometry the format cannot hold
                stats.unsupported += 1
                continue
        else:
            new = build(linear)
        setattr(parent, attr, new)
        if drop_original:
            linear.weight = None  # release the full-precision weight now
        stats.converted += 1
        stats.saved += saved_bytes(nbytes)
    return stats
