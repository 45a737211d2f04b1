"""logkv_amd: SemanticLogKV's flush-time compression path as HIP kernels for MI355X (gfx950).

Host surface mirrors the reference modules (litgpt/log_kv_cache.py,
litgpt/alpha_log_kv.py, litgpt/beta_log_kv.py, litgpt/log_kv_pack.py);
compute runs in liblogkv_hip.so through the C ABI in include/logkv_hip.h.
"""

from .log_kv_cache import (CacheAttentionState, LogKVStreamTrainingAttention, LogStructuredKVCache,  # noqa: F401
                           ladder_budget)
from .log_kv_pack import (append_exact_tokens, log_kv_chunk_attention, log_kv_slot_attention,  # noqa: F401
                          pack_mid_kv, packed_dim)
from . import beta_log_kv  # noqa: F401
from .kv_compression import cache_compression_snapshot, summarize_compression  # noqa: F401
from .streaming import LogKVStreamingAttention  # noqa: F401
from .flush_group import flush_grouping, set_flush_grouping  # noqa: F401
