"""Host-side contract of the drop-in classes (CPU only, no GPU compute)."""

from __future__ import annotations

import pytest
import torch


def test_constructor_argument_errors_precede_device_use() -> None:
    from saint_kv import kv_cache as kv

    with pytest.raises(ValueError, match="max_seq_len"):
        kv.SWAKVCacheLayer(max_seq_len=0, head_dim=8)
    with pytest.raises(ValueError, match="max_seq_len"):
        kv.HCAKVCacheLayer(max_seq_len=0, hidden_dim=8, head_dim=4, compression_rate=2)
    with pytest.raises(ValueError, match="compression_rate"):
        kv.HCAKVCacheLayer(max_seq_len=8, hidden_dim=8, head_dim=4, compression_rate=0)
    with pytest.raises(ValueError, match="compression_rate"):
        kv.CSAKVCacheLayer(max_seq_len=8, hidden_dim=8, head_dim=4, c_indexer=4, compression_rate=0)


def test_cpu_device_is_refused_loudly() -> None:
    from saint_kv import kv_cache as kv

    with pytest.raises(RuntimeError, match="ROCm GPU"):
        kv.SWAKVCacheLayer(max_seq_len=8, head_dim=8, device="cpu")
    if not torch.cuda.is_available():
        with pytest.raises(RuntimeError, match="ROCm GPU"):
            kv.SWAKVCacheLayer(max_seq_len=8, head_dim=8)


def test_ops_refuse_cpu_tensors() -> None:
    from saint_kv import ops

    pool = torch.zeros(4, 4, 8)
    bt = torch.zeros(1, 2, dtype=torch.int32)
    lens = torch.zeros(1, dtype=torch.int32)
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        ops.paged_gather(pool, bt, lens, torch.zeros(1, 8, 8))


def test_bundle_is_pure_plumbing() -> None:
    from saint_kv import kv_cache as kv

    bundle = kv.KVCacheBundle([None, None])
    assert len(bundle) == 2 and bundle.length == 0 and bundle.for_layer(1) is None
    bundle.reset()


def test_decode_descriptor_layout_matches_library() -> None:
    from saint_kv import decode

    decode.check_struct_layout()


def test_for_model_maps_subclasses_like_isinstance() -> None:
    """for_model matches the attention classes along the MRO, in the
    reference's isinstance order (kv_cache.py:395-426): subclasses of SWAttention,
    HCA and CSA map to their cache layer, other modules to None."""
    from saint_kv.kv_cache import _attention_kind

    class SWAttention:
        pass

    class HCA:
        pass

    class CSA:
        pass

    class WrappedCSA(CSA):
        pass

    class DeepHCA(type("Mid", (HCA,), {})):
        pass

    class Both(SWAttention, CSA):  # the isinstance chain tests SWAttention first
        pass

    class Dense:
        pass

    kinds = [_attention_kind(x()) for x in (SWAttention, HCA, CSA, WrappedCSA, DeepHCA, Both, Dense)]
    assert kinds == ["SWAttention", "HCA", "CSA", "CSA", "HCA", "SWAttention", None]
