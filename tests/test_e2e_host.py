"""The TTT model's data format and meta-step plumbing on the CPU (no GPU):
the key-value batches follow the reference's layout
(cloud_ttt_e2e/ttt_e2e/data.py), checked by decoding them, and the
parameter filter and chunking of the meta step (meta.py:9-41)."""
import pytest
import torch

from ttt_e2e import data, meta
from ttt_e2e.model import ModelConfig, TTTModel


@pytest.mark.parametrize("far", [0.0, 0.5])
def test_kv_batch_decodes(far):
    g = torch.Generator().manual_seed(1)
    bt = data.generate_kv_batch(3, 60, 30, 128, num_keys=16, device="cpu", pad_to=100, far_frac=far, generator=g)
    assert bt.input_ids.shape == bt.targets.shape == bt.inner_mask.shape == (3, 100)
    for b in range(3):
        seq = torch.cat([bt.input_ids[b, :1], bt.targets[b]]).tolist()
        assert seq[0] == data.BOS
        pairs = [seq[1 + 5 * i: 6 + 5 * i] for i in range(12)]
        assert all(p[0] == data.KEY and p[2] == data.VAL and p[4] == data.SEP for p in pairs)
        mapping = {p[1]: p[3] for p in pairs}
        assert len(mapping) == 12  # distinct keys
        assert all(6 <= k < 22 for k in mapping) and all(22 <= v < 38 for v in mapping.values())
        queries = [seq[61 + 5 * i: 66 + 5 * i] for i in range(6)]
        for q in queries:
            assert q[0] == data.QRY and q[2] == data.VAL and q[4] == data.SEP and mapping[q[1]] == q[3]
            if far:
                assert q[1] in [p[1] for p in pairs[:6]]  # drawn from the first far_frac share
        assert seq[91:] == [data.PAD] * 10
        # inner mask: targets inside the context; outer mask: the queries' value tokens
        assert bt.inner_mask[b].nonzero().flatten().tolist() == list(range(60))
        outer = bt.outer_mask[b].nonzero().flatten().tolist()
        assert outer == [60 + 5 * i + 3 for i in range(6)]
        assert all(bt.targets[b, i].item() == queries[(i - 63) // 5][3] for i in outer)


def test_param_filter_and_chunks():
    torch.manual_seed(0)
    cfg = ModelConfig(vocab_size=32, max_seq_len=64, window_size=16, d_model=32, n_heads=2, n_layers=3, d_ff=64,
                      suffix_layers=1)
    m = TTTModel(cfg)
    names = [n for n, _ in m.named_parameters()]
    chosen = meta.adapted_names(m, "mlp_fast")
    assert chosen and all("mlp_fast" in n for n in chosen)
    assert meta.adapted_names(m, None) == names
    assert meta.adapted_names(m, "nothing_matches") == names
    assert meta.adapted_names(m, " mlp_fast , ln_f ") == [n for n in names if "mlp_fast" in n or "ln_f" in n]
    assert meta.adapted_names(m, ["mlp_fast", "ln_f"]) == [n for n in names if "mlp_fast" in n or "ln_f" in n]
    assert meta._spans(48, 16) == [(0, 16), (16, 32), (32, 48)] and meta._spans(50, None) == [(0, 50)]
    with pytest.raises(ValueError):
        meta._spans(50, 16)
    assert len(m.prefix_blocks) == 2 and len(m.suffix_blocks) == 1 and hasattr(m.suffix_blocks[0], "mlp_slow")
    # reference parameter names (model.py): embed, pos, prefix_blocks.i.{ln1,attn.*_proj,ln2,mlp}, suffix ...
    for n in ("embed.weight", "pos.weight", "prefix_blocks.0.attn.q_proj.weight", "prefix_blocks.1.mlp.2.bias",
              "suffix_blocks.0.mlp_fast.0.weight", "suffix_blocks.0.mlp_slow.2.weight", "ln_f.weight",
              "head.weight"):
        assert n in names, n
    assert "head.bias" not in names
    with pytest.raises(ValueError):
        m(None, mode="full")
    with pytest.raises(ValueError):
        m(None, mode="suffix")
