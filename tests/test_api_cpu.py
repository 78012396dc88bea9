"""CPU checks of the drop-in API's host logic (no kernel launches): argument rules the
reference enforces, shape rules of this build, and that the product path refuses to run
without device tensors instead of falling back to a CPU implementation."""
import pytest
import torch

import modules
from modules import _hip


def test_exports():
    for name in ("WindowBuffer", "RetrievalIndex", "TileKVCache", "KVRHook", "KVRGenerator"):
        assert hasattr(modules, name)


def test_retrieval_append_requires_calibrate():
    """kvr_retrieval.py:164-165: append before calibrate raises RuntimeError."""
    ri = modules.RetrievalIndex(2, 128, device="cpu")
    with pytest.raises(RuntimeError, match="calibrate"):
        ri.append(torch.zeros(2, 128))


def test_retrieval_empty_returns():
    ri = modules.RetrievalIndex(2, 128, device="cpu")
    k, v = ri.retrieve_topk(torch.zeros(8, 128))
    assert k.shape == (0, 2, 128) and v.shape == (0, 2, 128)
    assert ri.compute_chunk_scores(torch.zeros(8, 128)).shape == (0, 2)
    assert ri.build_attractors() is None


def test_head_dim_must_be_128():
    with pytest.raises(ValueError):
        modules.RetrievalIndex(2, 64, device="cpu")
    with pytest.raises(ValueError):
        modules.WindowBuffer(2, 64, device="cpu")
    from transformers import LlamaConfig, LlamaForCausalLM
    cfg = LlamaConfig(vocab_size=64, hidden_size=128, intermediate_size=128, num_hidden_layers=1,
                      num_attention_heads=2, num_key_value_heads=1)
    with pytest.raises(ValueError, match="head_dim 128"):
        modules.KVRHook(LlamaForCausalLM(cfg), device="cpu")


def test_cache_shape_rules():
    with pytest.raises(ValueError, match="multiple"):
        modules.TileKVCache(1, 2, 100, 64, _hip.HADAMARD, "cpu")
    with pytest.raises(ValueError, match="unsupported"):
        modules.TileKVCache(1, 2, 96, 32, _hip.HADAMARD, "cpu")


def test_window_ring_semantics_cpu():
    """append / batch_append ring bookkeeping (kvr_window.py:19-41) is host-side tensor work."""
    wb = modules.WindowBuffer(1, 128, window_size=8, device="cpu")
    k = torch.arange(20, dtype=torch.float32)[:, None, None].expand(20, 1, 128)
    wb.batch_append(k[:5], k[:5])
    assert (wb.pos, wb.n) == (5, 5)
    wb.batch_append(k[5:13], k[5:13])
    assert (wb.pos, wb.n) == (13, 8)
    wb.append(k[13], k[13])
    assert sorted(wb.k[:, 0, 0].tolist()) == list(range(6, 14))


def test_product_path_refuses_cpu_tensors():
    wb = modules.WindowBuffer(1, 128, window_size=8, device="cpu")
    wb.append(torch.ones(1, 128), torch.ones(1, 128))
    with pytest.raises(RuntimeError, match="device tensors"):
        wb.attention(torch.ones(2, 128))
    c = modules.TileKVCache(1, 2, 64, 64, _hip.HADAMARD, "cpu")
    with pytest.raises(RuntimeError, match="device tensors"):
        c.load_prompt(torch.zeros(1, 2, 200, 128), torch.zeros(1, 2, 200, 128))
