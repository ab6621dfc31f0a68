"""The C-ABI library loads and exports every entry point its header declares.

Host-only: no device memory is touched and no kernel is launched.
"""
from __future__ import annotations

import ctypes
import re
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "helix_kv.h"


def declared_functions() -> list[str]:
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b(hkv_\w+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    from helix_kv import _native

    L = _native.lib()
    names = declared_functions()
    assert len(names) >= 16
    missing = [n for n in names if not hasattr(L, n)]
    assert not missing, missing
    # the Python binding declares a signature for every exported entry point
    assert sorted(_native.exported_symbols()) == names


def test_host_only_entry_points():
    from helix_kv import _native

    L = _native.lib()
    assert b"gfx950" in L.hkv_version()
    assert L.hkv_status_string(0) == b"ok"
    assert L.hkv_status_string(4) == b"output capacity too small"
    # 256-byte header (work counter, finished waves, epoch, error word), then
    # one 8-byte status word per chunk (four waves of at least 64 rows)
    # a 256-byte header and 8 bytes per chunk of 256 rows, for at least 2048
    # chunks (a small tensor is packed in smaller chunks)
    assert L.hkv_nuq_pack_compact_workspace_bytes(262144, 4, 128) == 256 + 8 * (262144 * 4 // 256)
    assert L.hkv_nuq_pack_compact_workspace_bytes(131072, 4, 128) == 256 + 8 * 2048
    assert L.hkv_nuq_pack_compact_workspace_bytes(10, 4, 128) == 256 + 8 * 2048
    assert L.hkv_nuq_pack_compact_workspace_bytes(0, 4, 128) == 256 + 8 * 2048
    assert L.hkv_nuq_pack_compact_workspace_bytes(10, 4, 100) == 0  # unsupported D
    assert L.hkv_quest_topk_workspace_bytes(65536, 4) >= 64


def test_struct_layouts_match_header():
    from helix_kv import _native

    assert ctypes.sizeof(_native.NuqScales) == 4 * 8 + 4 * 4 + 8 + 8 + 8
    assert ctypes.sizeof(_native.TensorDesc) == 8 + 4 + 4 + 6 * 8
    # hkv_pack_item: values, T, H/D/bits/reserved, scales, 4 pointers, capacity
    assert ctypes.sizeof(_native.PackItem) == 8 + 8 + 16 + ctypes.sizeof(_native.NuqScales) + 32 + 8
    assert _native.PackItem.scales.offset == 32
    assert "#define HKV_TABLE_BYTES 80" in HEADER.read_text()
    assert _native.TABLE_BYTES == 80


def test_oracle_table_record_matches_device_layout():
    import oracle

    assert oracle.TABLE_DTYPE.itemsize == 80
    assert oracle.TABLE_DTYPE.fields["lo"][1] == 64
    assert oracle.TABLE_DTYPE.fields["xsafe"][1] == 68
    assert oracle.TABLE_DTYPE.fields["flags"][1] == 70
