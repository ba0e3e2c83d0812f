"""Dense ``[S * H]`` masks from the reference's token-head arguments.

``PackedKVCache.evict(set)``, ``PackedKVCache.apply_reuse_mask(dict)`` and
``PagedKVStore.evict_tokens(set)`` take a Python set of ``(token, head)``
pairs, or a dict ``(token, head) -> flag``, and the reference tests each entry
with ``in`` / ``.get`` (packed_kv_cache.py:679-687, 798-814;
paged_kv_store.py:618-632). The kernels take a uint8 mask instead; one pass
over the container fills it with the same rule: an item marks entry
``t * H + h`` when it equals the tuple ``(t, h)`` for an in-range token and
head (for a dict, when its value is truthy too).

The pass runs in the host extension ``_hostmask`` (csrc/host_masks.c) for ints,
floats and numpy integers; other element types, or a missing extension, take
the item-by-item Python rule below, which gives the same result.
"""

from __future__ import annotations

import importlib.machinery
import importlib.util
import os
import sysconfig
import threading
from itertools import compress
from typing import Any, Optional

import numpy as np

_lock = threading.Lock()
_mod: Any = None
_tried = False


def _ext():
    global _mod, _tried
    if not _tried:
        with _lock:
            if not _tried:
                path = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))),
                                    "_lib", "_hostmask" + (sysconfig.get_config_var("EXT_SUFFIX")
                                                           or ".so"))
                if os.path.exists(path):
                    loader = importlib.machinery.ExtensionFileLoader("_hostmask", path)
                    spec = importlib.util.spec_from_file_location("_hostmask", path, loader=loader)
                    mod = importlib.util.module_from_spec(spec)
                    loader.exec_module(mod)
                    _mod = mod
                _tried = True
    return _mod


def _entry(item, S: int, H: int) -> Optional[int]:
    """``t * H + h`` when ``item`` equals the in-range pair ``(t, h)`` (Python's
    own tuple equality: 3.0 matches 3, 3.5 and "3" match nothing), else None."""
    if not isinstance(item, tuple) or len(item) != 2:
        return None
    try:
        t, h = int(item[0]), int(item[1])
    except (TypeError, ValueError, OverflowError):
        return None
    if (t, h) == item and 0 <= t < S and 0 <= h < H:
        return t * H + h
    return None


def _mark_python(items, S: int, H: int, out: np.ndarray, is_dict: bool) -> int:
    """Item by item; a dict value's truthiness is evaluated only for in-range
    pairs (the reference evaluates ``reuse_mask.get(entry)`` only for entries
    of the cache, packed_kv_cache.py:797-799)."""
    marked = 0
    for item, value in (items.items() if is_dict else ((i, True) for i in items)):
        e = _entry(item, S, H)
        if e is not None and value:
            out[e] = 1
            marked += 1
    return marked


def token_head_mask(items, S: int, H: int, is_dict: bool = False) -> Optional[np.ndarray]:
    """uint8 ``[S * H]`` mask of the pairs in ``items`` (a set or other
    iterable of pairs; with ``is_dict``, the keys whose value is truthy), or
    None when no in-range pair is marked."""
    out = np.zeros(S * H, dtype=np.uint8)
    mod = _ext()
    marked = None
    if mod is not None and (not is_dict or isinstance(items, dict)):
        marked = mod.token_head_mask(items, S, H, out, bool(is_dict))
    if marked is None:
        out[:] = 0
        marked = _mark_python(items, S, H, out, is_dict)
    return out if marked else None
