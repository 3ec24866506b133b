"""q3attn: MI355X (gfx950) attention for the Qwen3-TTS engine's hot path.

Entry points (each a drop-in for the reference call it names):
  * ``flash_attn_with_kvcache`` / ``paged_decode``  -- talker decode attention (engine/talker.py:77)
  * ``paged_decode_append`` (``k=``/``v=`` form)   -- KV append + decode (engine/talker.py:72-73, :77)
  * ``paged_decode_append_rope``                     -- q/k RMSNorm + RoPE, KV append and decode (engine/talker.py:69-77)
  * ``cp_attn`` / ``cp_attn_append``                 -- code-predictor attention (engine/cp_attn.py:33-39;
                                                       slot write fused: engine/code_predictor.py:58)
  * ``cp_attn_append_rope``                          -- + the step's q/k norm and RoPE (engine/code_predictor.py:38-43)
  * ``flash_attn_varlen_func`` / ``flash_attn_func``  -- prefill (engine/talker.py:169, engine/arrivals.py:148)
  * ``prefill_append``                               -- prompt K/V into the pool + prefill (engine/talker.py:161-169)
  * ``prefill_append_rope``                          -- + the prompt's q/k norm and RoPE (engine/talker.py:157-169)
  * ``prefill_dense_append``                         -- admission K/V into the pool + prefill (engine/arrivals.py:144-148)
  * ``prefill_dense_append_rope``                    -- + the admission q/k norm, RoPE and K/V concat (engine/arrivals.py:112-118)
  * ``PagePool``                                     -- 16-token pages per seat from a free list, device block table
"""
import torch  # noqa: F401  (loads the HIP runtime the library binds to)

from ._lib import LIB_PATH, Q3AttnError, lib  # noqa: F401
from .cp_attn import (cp_attn, cp_attn_append, cp_attn_append_op, cp_attn_append_rope,  # noqa: F401
                      cp_attn_append_rope_op, cp_attn_op)
from .ops import (DECODE_CHUNKS, DECODE_PLANNED, DECODE_ROW, DECODE_STREAMK, decode_plan,  # noqa: F401
                  flash_attn_with_kvcache, paged_decode,  # noqa: F401
                  paged_decode_append, paged_decode_append_rope)
from .pages import PagePool, PoolExhausted  # noqa: F401
from .prefill import (flash_attn_func, flash_attn_varlen_func, prefill, prefill_append, prefill_dense,  # noqa: F401
                      prefill_append_rope, prefill_dense_append, prefill_dense_append_rope)
