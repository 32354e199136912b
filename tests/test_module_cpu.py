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
