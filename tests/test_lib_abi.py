"""The C-ABI library loads and exports exactly what include/pagedkv.h declares (CPU only:
loading the library and resolving symbols makes no GPU call)."""
import ctypes
import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "pagedkv.h"


def _declared():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b(pkv_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_entry_points():
    names = _declared()
    assert "pkv_batch_decode" in names and "pkv_append_paged_kv_cache" in names
    assert len(names) >= 8


def test_library_exports_every_declared_symbol():
    from ecahlang_amd import _lib

    h = _lib.lib()
    missing = [n for n in _declared() if not hasattr(h, n)]
    assert not missing, missing


def test_python_signatures_cover_header():
    from ecahlang_amd import _lib

    assert sorted(_lib.SIGNATURES) == _declared()


def _declared_arity():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    out = {}
    for m in re.finditer(r"\b(pkv_[a-z0-9_]+)\s*\(([^;]*?)\)\s*;", text, flags=re.S):
        params = m.group(2).strip()
        out[m.group(1)] = 0 if params in ("", "void") else params.count(",") + 1
    return out


def test_python_argument_counts_match_header():
    # a binding with the wrong number of arguments would pass garbage to the library on the GPU
    from ecahlang_amd import _lib

    arity = _declared_arity()
    assert sorted(arity) == _declared()
    wrong = {n: (len(_lib.SIGNATURES[n][1]), k) for n, k in arity.items() if len(_lib.SIGNATURES[n][1]) != k}
    assert not wrong, wrong


def test_loader_refuses_missing_library(monkeypatch, tmp_path):
    from ecahlang_amd import _lib

    monkeypatch.setattr(_lib, "_LIB", None)
    monkeypatch.setattr(_lib, "LIB_PATH", tmp_path / "nope.so")
    with pytest.raises(RuntimeError, match="no CPU or PyTorch fallback"):
        _lib.lib()


def test_workspace_sizing_is_host_only():
    from ecahlang_amd import _lib

    n = _lib.lib().pkv_decode_workspace_bytes(64, 16, 128, 256, 12000)
    assert n >= (256 + 64) * 16 * 128 * 4
    assert _lib.lib().pkv_decode_uses_mfma(0, 128, 16, 2, 64) == 1
    assert _lib.lib().pkv_decode_uses_mfma(2, 64, 32, 8, 4) == 0
    # no batch limit (the schedule replaces the page-table rows staged in LDS)
    assert _lib.lib().pkv_decode_uses_mfma(0, 128, 16, 2, 4096) == 1
    # head blocks: 32 KV heads of head_dim 128 at group 1 are 16 blocks of two, over the 8 waves
    assert _lib.lib().pkv_decode_uses_mfma(0, 128, 32, 32, 4) == 0
    assert _lib.lib().pkv_decode_uses_mfma(1, 128, 32, 8, 4) == 1


def test_split_partial_ml_slots_are_whole_cache_lines():
    # Each split segment's (max, sum) slot covers whole 128-byte lines (16 float2), so a merger
    # never pulls another sequence's slot into its L2 before that slot is written.  Between
    # 8 and 16 q heads the (max, sum) area must not grow; only the partial rows (D floats per
    # head and slot) do.
    from ecahlang_amd import _lib

    a256 = lambda x: -(-x // 256) * 256
    batch, d, ctas, nidx = 64, 128, 256, 12000
    slots = max(ctas, -(-nidx // 512)) + batch
    ws = lambda hq: _lib.lib().pkv_decode_workspace_bytes(batch, hq, d, ctas, nidx)
    for hq in range(9, 17):
        assert ws(hq) - ws(hq - 1) == a256(slots * hq * d * 4) - a256(slots * (hq - 1) * d * 4)
    # crossing a multiple of 16 heads adds exactly one line per slot
    assert ws(17) - ws(16) == (a256(slots * 17 * d * 4) - a256(slots * 16 * d * 4)
                               + a256(slots * 32 * 8) - a256(slots * 16 * 8))


def test_flashinfer_namespace_covers_reference_call_sites():
    import ecahlang_amd.fi as flashinfer

    for name in ("get_seq_lens", "get_batch_indices_positions", "BatchDecodeWithPagedKVCacheWrapper",
                 "BatchPrefillWithPagedKVCacheWrapper"):
        assert callable(getattr(flashinfer, name))
    assert callable(flashinfer.page.append_paged_kv_cache)
    assert callable(flashinfer.sampling.top_k_top_p_sampling_from_logits)


def test_attention_hook_registers_with_transformers():
    from transformers import AttentionInterface

    from ecahlang_amd import hook

    hook.register()
    assert AttentionInterface._global_mapping.get(hook.HOOK_NAME) is hook.ecah_attention


def test_noalloc_decode_refuses_geometry_beyond_its_array():
    # A page list long enough to need more ranges than the 16 MiB array holds: refused with the
    # workspace error before anything is enqueued (no device call is made, so this runs on the
    # CPU with null pointers).
    from ecahlang_amd import _lib

    L = _lib.lib()
    assert L.pkv_decode_workspace_bytes(64, 16, 128, 256, 10_000_000) > (16 << 20)
    rc = L.pkv_batch_decode_noalloc(None, 0, 0, None, None, 0, 0, None, None, 10_000_000, None, 64, 16, 2, 128,
                                    16, 0.1, 256, None, 0, 0, 0, None)
    assert rc == -6
