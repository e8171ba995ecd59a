"""Run-time inference settings, read when a call needs them rather than at import.

The reference keeps these in `default_config.INFERENCE` (default_config.py:1684-1700) and lets a
run override them with `--set INFERENCE.key=value`; here a caller edits the dict itself, e.g.
`mira_amd.config.INFERENCE["prefix_cache"] = 0`, and every later call sees the new value.

  prefix_cache       1 lets inference forwards carry lattice state in a PrefixCache; 0 makes the
                     mixer refuse a cache. Training never passes one.
  prefix_cache_size  the most a PrefixCache may hold, in GiB (0 = no ceiling). The state has a
                     fixed size per sequence, so this bounds the batch, not the context.
  max_context        the context length an HF-style wrapper reports (a ceiling, not a property of
                     the model: nothing in it refers to an absolute position).
"""
from __future__ import annotations

INFERENCE = {"prefix_cache": 1, "prefix_cache_size": 2, "max_context": 262144}
