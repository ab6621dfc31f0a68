"""helix_kv -- MI355X-native (gfx950) KV-cache hot path for helix-lite.

The drop-in Python surface lives in the sibling packages ``kvquant`` and
``quest`` (same module paths and signatures as the reference's ``src/``);
this package holds the native binding and the operations they share.
"""
from . import _native  # noqa: F401
from .ops import (  # noqa: F401
    NuqLayerTables,
    build_tables,
    nuq_pack_dense,
    nuq_unpack_dense,
    nuq_pack_compact,
    nuq_unpack_compact,
    CompactCodes,
    quest_page_stats,
    quest_page_bound,
    quest_topk,
    quest_select,
)


def version() -> str:
    return _native.lib().hkv_version().decode()
