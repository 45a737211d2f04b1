"""logkv_amd: SemanticLogKV's flush-time compression path as HIP kernels for MI355X (gfx950).

Host surface mirrors the reference modules (litgpt/log_kv_cache.py,
litgpt/alpha_log_kv.py, litgpt/beta_log_kv.py, litgpt/log_kv_pack.py);
compute runs in liblogkv_hip.so through the C ABI in include/logkv_hip.h.
"""

from .log_kv_cache import LogStructuredKVCache, ladder_budget  # noqa: F401
from .log_kv_pack import log_kv_chunk_attention, pack_mid_kv, packed_dim  # noqa: F401
from .kv_compression import cache_compression_snapshot, summarize_compression  # noqa: F401
from .streaming import LogKVStreamingAttention  # noqa: F401
