"""Host-side behaviour of the drop-in module (CPU only): the reference's
constructor errors (elastic_sparse_attention.py:412-417, :435-441), its
attributes (:425-444), and no silent CPU path."""
import pytest
import torch

from elastic_sparse_attention import ElasticSparseAttention


def test_constructor_attributes():
    m = ElasticSparseAttention(layer_idx=4, num_hidden_layers=8, num_attention_heads=32,
                               head_dim=128, attention_length=64, max_seq_len=32768)
    assert m.scaling == 128 ** -0.5
    assert m.num_key_value_heads == 32 and m.num_kv_groups == 1
    assert m.implementation == "triton"
    g = ElasticSparseAttention(1, 8, 32, 64, 64, 4096, num_key_value_heads=8,
                               implementation="naive")
    assert g.num_kv_groups == 4 and g.implementation == "naive"
    assert list(m.parameters()) == [] and m.state_dict() == {}


def test_invalid_implementation():
    with pytest.raises(ValueError, match="Invalid implementation"):
        ElasticSparseAttention(0, 8, 4, 64, 64, 1024, implementation="cuda")


def test_gqa_divisibility():
    with pytest.raises(ValueError, match="must be divisible"):
        ElasticSparseAttention(0, 8, 6, 64, 64, 1024, num_key_value_heads=4)


def test_cpu_tensors_raise():
    m = ElasticSparseAttention(0, 8, 4, 64, 64, 1024)
    q = torch.randn(1, 4, 16, 64)
    with pytest.raises(RuntimeError, match="GPU"):
        m(q, q, q)


def test_index_buffers_registered_like_the_reference():
    """The reference registers its index buffers as non-persistent buffers
    (:454-468): here too, so they stay out of the state dict and follow
    module.to(); they are None until first read (the kernels never read
    them), and "dense" registers full_attention_mask instead."""
    m = ElasticSparseAttention(4, 8, 4, 64, 64, 1024)
    names = set(m._buffers)
    assert {"sparse_attention_indices", "sparse_causal_mask", "full_attention_mask"} <= names
    assert m._buffers["sparse_attention_indices"] is None
    assert m.state_dict() == {}
    assert m.to(torch.float32) is m
    if not torch.cuda.is_available():
        # the builders are HIP kernels: no CPU path to fall back to
        with pytest.raises(RuntimeError, match="GPU"):
            m.sparse_attention_indices
        d = ElasticSparseAttention(4, 8, 4, 64, 64, 1024, implementation="dense")
        assert d.sparse_attention_indices is None
        with pytest.raises(RuntimeError, match="GPU"):
            d.full_attention_mask
