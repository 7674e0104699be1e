"""MI355X-native (gfx950) depth-aware paged-KV hot path for looped LMs.

A drop-in "hip" backend for vllm_rlt's KV-cache manager and attention-backend
interfaces, backed by hand-written HIP kernels in librlt_kv.so (C ABI in
include/rlt_kv.h).
"""

from . import ops
from .async_state import AsyncState, RoutingBank
from .buffers import Workspace
from .device_cache import DeviceCache
from .graphs import RecurrentGraphs
from .kv_cache_manager import KVCacheManager
from .page_book import KVPageBook, PreparedKVBatch
from .paged_attention import HipPagedAttention, hip_paged_attention
from .prefill_metadata import PrefillMetadataBank
from .prefill_order import PrefillItem, PrefillOrder

__all__ = [
    "AsyncState",
    "DeviceCache",
    "HipPagedAttention",
    "KVCacheManager",
    "KVPageBook",
    "PrefillItem",
    "PrefillMetadataBank",
    "PrefillOrder",
    "PreparedKVBatch",
    "RecurrentGraphs",
    "RoutingBank",
    "Workspace",
    "hip_paged_attention",
    "ops",
]
