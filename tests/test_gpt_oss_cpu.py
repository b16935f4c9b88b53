"""CPU tests of the GPT-OSS adapter's host logic (gpt_oss.py): what it reads from a padding mask
or from position ids, that it reads it once per batch, and how packed rows are routed.  The
varlen attention call is replaced, inside these tests only, by a recorder; no kernel runs."""
import pytest
import torch

from conftest import load_mod

gpt_oss = load_mod("gpt_oss")


def test_mask_facts_padded_and_full():
    m = torch.tensor([[1, 1, 1, 0, 0], [0, 1, 1, 1, 1]], dtype=torch.bool)
    full, idx, cu, max_len = gpt_oss._mask_facts(m)
    assert not full
    assert idx.tolist() == [0, 1, 2, 6, 7, 8, 9]
    assert cu.tolist() == [0, 3, 7] and cu.dtype == torch.int32
    assert max_len == 4
    assert gpt_oss._mask_facts(torch.ones(2, 5, dtype=torch.long))[0] is True


def test_position_facts_packed_row():
    # three sequences of 4, 2 and 3 tokens packed into one row
    p = torch.tensor([[0, 1, 2, 3, 0, 1, 0, 1, 2]])
    cu, max_len = gpt_oss._position_facts(p)
    assert cu.tolist() == [0, 4, 6, 9] and cu.dtype == torch.int32
    assert max_len == 4
    # ids that start above 0 restart at their minimum (transformers' rule)
    cu, _ = gpt_oss._position_facts(p + 2)
    assert cu.tolist() == [0, 4, 6, 9]
    # one increasing run, or more than one row: not packed
    assert gpt_oss._position_facts(torch.arange(7).unsqueeze(0)) is None
    assert gpt_oss._position_facts(torch.arange(7).unsqueeze(0) + 5) is None
    assert gpt_oss._position_facts(torch.stack([torch.arange(4), torch.tensor([0, 1, 0, 1])])) is None


def test_batch_facts_are_computed_once_per_tensor():
    facts = gpt_oss._BatchFacts()
    calls = []

    def compute(t):
        calls.append(1)
        return int(t.sum())

    m = torch.ones(2, 3)
    assert facts.get(m, compute) == 6 and facts.get(m, compute) == 6
    assert len(calls) == 1  # the second layer reuses the first layer's facts
    m.zero_()  # modified in place: recomputed
    assert facts.get(m, compute) == 0 and len(calls) == 2
    m2 = torch.ones(2, 3)  # another batch
    assert facts.get(m2, compute) == 6 and len(calls) == 3


@pytest.fixture
def varlen_recorder(monkeypatch):
    seen = []

    def fake(q, k, v, cu, max_len, W, S, scale, sinks):
        seen.append(dict(q=q.shape, k=k.shape, cu=cu.tolist(), max_len=max_len, W=W, S=S, scale=scale))
        return torch.zeros_like(q)

    monkeypatch.setattr(gpt_oss, "flash_swda_with_sink_varlen", fake)
    return seen


def test_packed_position_ids_run_as_a_packed_batch(varlen_recorder):
    B, Hq, Hkv, L, D = 1, 4, 2, 9, 16
    q, k, v = torch.zeros(B, Hq, L, D), torch.zeros(B, Hkv, L, D), torch.zeros(B, Hkv, L, D)
    pos = torch.tensor([[0, 1, 2, 3, 0, 1, 0, 1, 2]])
    o, w = gpt_oss.gpt_oss_attention_forward(None, q, k, v, None, scaling=0.25, sliding_window=3, position_ids=pos)
    assert w is None and o.shape == (B, L, Hq, D)
    assert varlen_recorder == [dict(q=(L, Hq, D), k=(L, Hkv, D), cu=[0, 4, 6, 9], max_len=4, W=3, S=0, scale=0.25)]
    # a full layer (no window) uses the longest sequence as its window
    gpt_oss.gpt_oss_attention_forward(None, q, k, v, None, scaling=0.25, sliding_window=None, position_ids=pos)
    assert varlen_recorder[-1]["W"] == 4


def test_collator_offsets_run_as_a_packed_batch(varlen_recorder):
    B, Hq, Hkv, L, D = 1, 2, 1, 6, 16
    q, k, v = torch.zeros(B, Hq, L, D), torch.zeros(B, Hkv, L, D), torch.zeros(B, Hkv, L, D)
    cu = torch.tensor([0, 2, 6], dtype=torch.int32)
    gpt_oss.gpt_oss_attention_forward(None, q, k, v, None, sliding_window=128, cu_seq_lens_q=cu, cu_seq_lens_k=cu,
                                      max_length_q=4, max_length_k=4)
    assert varlen_recorder[-1]["cu"] == [0, 2, 6] and varlen_recorder[-1]["max_len"] == 4
    with pytest.raises(NotImplementedError, match="cu_seq_lens_k differs"):
        gpt_oss.gpt_oss_attention_forward(None, q, k, v, None, cu_seq_lens_q=cu,
                                          cu_seq_lens_k=torch.tensor([0, 3, 6], dtype=torch.int32))


def test_unpacked_position_ids_take_the_plain_path(monkeypatch, varlen_recorder):
    plain = []
    monkeypatch.setattr(gpt_oss, "attention", lambda q, k, v, **kw: plain.append(kw) or torch.zeros_like(q))
    q = torch.zeros(1, 2, 5, 16)
    gpt_oss.gpt_oss_attention_forward(None, q, q[:, :1], q[:, :1], None, position_ids=torch.arange(5).unsqueeze(0))
    assert len(plain) == 1 and varlen_recorder == []
