"""MI355X-native serving hot path for Qwen3-TTS (gfx950 HIP kernels behind a C ABI).

Import this package after ``torch``.  Submodules:

- ``talker_kv``  -- PagedTalkerKV + HIP attention bindings (GPU planner, attention plan)
- ``cache``      -- host page ownership with pending/publish/discard publications
- ``kernels``    -- qk-norm/RoPE/KV-write and short-cache attention entry points
- ``sampling``   -- fused uniform-driven sampler and Philox uniforms
- ``layers``     -- fused add-RMSNorm, RMSNorm, SwiGLU
- ``talker``     -- one random-init talker decode step (the metric's unit)
- ``graphs``     -- hipGraph capture driver and bucket lowering
- ``build``      -- hipcc recipe for ``libnq_hip.so``
"""

from __future__ import annotations

import torch  # noqa: F401  (binds the HIP runtime before the library loads)

from . import _lib  # noqa: F401

__all__ = ["_lib"]
