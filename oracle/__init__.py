"""CPU oracle for the serving hot path -- TEST INFRASTRUCTURE ONLY.

This package restates, in numpy, the algorithms of nari-labs/nari-qwen3-tts
that the HIP kernels replace.  It checks the product and is never part of it: only
``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import it.  The product package fails loudly when its HIP
library is missing and never falls back to anything here.

Modules and what they restate (reference paths are relative to
``src/nari_qwen3_tts/``):

- ``planner``   -- PagedKVAllocator (executor/cache.py:86-212) and
                   PagedTalkerKV._metadata (executor/talker_kv.py:403-483)
- ``attention`` -- paged GQA decode / causal prefill and the short-cache
                   attention (executor/talker_kv.py:140-306,
                   model/kernels.py:408-463, model/components.py:235-252)
- ``qk_rope``   -- paired q/k RMSNorm + RoPE + cache write
                   (model/kernels.py:15-91, 163-248)
- ``sampler``   -- the uniform-driven sampler contract, Philox-4x32-10 and the
                   exp used by both sides (executor/sampling.py:242-302,
                   model/sampling.py:55-225)
- ``norms``     -- RMSNorm, residual add + RMSNorm, SwiGLU (model/layers.py:28-115)
- ``talker``    -- one talker decode step over the above (model/components.py:29-90,
                   executor/talker.py:231-262, 341-374)

Parity status of each function (pinned / unpinned) is recorded in the module
docstrings and in the tests that pin them.
"""
