"""mira_amd -- the Mira mixer scan on MI355X (gfx950): HIP kernels behind a C-ABI
(include/mira_hip.h, lib/libmira_hip.so) and the host mirror of the reference's plugin API.

  mira_amd.mira          the operator plugin (kernel/cuda/mira_dspv2/mira.py's API)
  mira_amd.hardware      device selection (kernel/hardware.py's API), HIP only
  mira_amd.prefix_cache  the decode-state cache (model/prefix_cache.py's API)
  mira_amd.mixer         MiraMixer with the reference constructor and forward signature
  mira_amd.block         RMSNorm, FeedForward and MiraBlock (model/mira_block.py's API)
  mira_amd.llm           MiraLLM, the stack of blocks between the tied embedding and head
  mira_amd.generate      decoding through the prefix cache (mirachat.generate's loop, batched)
"""
from . import mira  # noqa: F401
