"""GPU attention-hole checker (esa_reachability) against the oracle's
restatement of check_attn_hole.py:53-180: the reachable set bit for bit and
the set size after every layer."""
import pytest
import torch

from esa_oracle import attention_reachability as oracle_reach
from check_attn_hole import attention_reachability, check_attention_holes_pytorch

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)


@pytest.mark.parametrize("L,nl,H,w,pos", [
    (4096, 8, 8, 64, 4095),
    (4096, 8, 8, 16, 4095),
    (32768, 8, 8, 16, 32767),    # the reference's w = 16 example: holes remain
    (512, 12, 8, 32, 511),
    (1000, 3, 5, 7, 999),
    (200, 1, 4, 16, 100),        # one layer: the sliding window
    (128, 8, 8, 64, 0),          # position 0 sees only itself
    (2048, 8, 8, 64, 62),        # below w - 1: the whole prefix
    (300001, 6, 2, 16, 300000),  # more than one 262144-token LDS window
    (70000, 8, 3, 100, 69999),
])
def test_reachability_matches_oracle(L, nl, H, w, pos):
    print(f"reach L={L} nl={nl} H={H} w={w} pos={pos}", flush=True)
    r = attention_reachability(L, nl, H, w, pos, device=DEV)
    want, counts = oracle_reach(nl, H, w, pos)
    assert torch.equal(r.reachable.cpu(), want)
    assert r.layer_counts == counts
    assert r.holes == pos + 1 - counts[-1]


def test_reference_claims_at_131072(capsys):
    # check_attn_hole.py:182-220, theory/note.md:85: 8 layers, 8 heads,
    # w = 64 leave no hole at positions 131071 and 4095
    for pos in (131071, 4095):
        print(f"reach claim pos={pos}", flush=True)
        r = check_attention_holes_pytorch(131072, 8, 8, 64, position_id=pos)
        assert r.holes == 0 and bool(r.reachable.all())
        want, counts = oracle_reach(8, 8, 64, pos)
        assert r.layer_counts == counts
    out = capsys.readouterr().out
    assert "SUCCESS: Position 131071 has no attention holes" in out
    assert "SUCCESS: Position 4095 has no attention holes" in out


def test_report_lists_holes(capsys):
    r = check_attention_holes_pytorch(131072, 8, 8, 16, position_id=32767)
    out = capsys.readouterr().out
    assert r.holes > 0
    assert f"FAILURE: Position 32767 has {r.holes} attention holes" in out
    assert str(r.unreachable()[:10].tolist()) in out


def test_repeat_calls_are_identical():
    a = attention_reachability(50000, 8, 8, 32, 49999, device=DEV)
    b = attention_reachability(50000, 8, 8, 32, 49999, device=DEV)
    assert torch.equal(a.reachable, b.reachable) and a.layer_counts == b.layer_counts
