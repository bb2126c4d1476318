"""selector.targets on the host: the reference's loader contract
(selector/targets.py:21-123) without a GPU -- file contents, error messages,
and that pickled objects in a teacher file are refused (weights_only load)."""
import pytest
import torch

from selector.targets import causal_block_mask, load_selector_features, load_teacher

L, G, H, QB, P, D = 2, 2, 6, 5, 3, 8


def _teacher_dict(seed=0, proto=True, pooled=True, dtype=torch.bfloat16):
    g = torch.Generator().manual_seed(seed)
    d = {
        "pooledQ": torch.randn(1, L, G, QB, P, D, generator=g).to(dtype),
        "pooledK": torch.randn(1, L, G, QB, P, D, generator=g).to(dtype),
        "seq_len": 300, "block_size": 64, "proto": P if proto else None,
        "needle_block": 2, "prompt_format": "plain", "dense_screen": {"accepted": True},
        "case_id": "c0", "depth": 0.5, "rope": {"theta": 1e6},
    }
    if pooled:
        d["pooled"] = torch.rand(1, L, H, QB, QB, generator=g)
    return d


def test_selector_features_shapes_and_meta(tmp_path):
    path = tmp_path / "t.pt"
    torch.save(_teacher_dict(), path)
    out = load_selector_features(path)
    assert out["q_feat"].shape == (L, G, QB, P, D) and out["q_feat"].dtype == torch.float32
    assert out["k_feat"].shape == (L, G, QB, P, D)
    m = out["meta"]
    assert set(m) == {"seq_len", "block_size", "requested_length", "needle_block", "num_layers", "num_groups",
                      "qb", "kb", "head_dim", "proto", "rope", "features_only", "prompt_format",
                      "dense_screen_accepted", "case_id", "depth"}
    assert (m["seq_len"], m["requested_length"], m["num_layers"], m["num_groups"], m["qb"], m["proto"]) == \
        (300, 300, L, G, QB, P)
    assert m["dense_screen_accepted"] is True and m["rope"] == {"theta": 1e6}


def test_reference_error_messages(tmp_path):
    path = tmp_path / "old.pt"
    torch.save(_teacher_dict(proto=False), path)
    with pytest.raises(KeyError, match="lacks P-prototype selector features"):
        load_selector_features(path)
    with pytest.raises(KeyError, match="predates multi-prototype extraction"):
        load_teacher(path)
    path2 = tmp_path / "features.pt"
    torch.save(_teacher_dict(pooled=False), path2)
    with pytest.raises(ValueError, match="selector-feature-only artifact"):
        load_teacher(path2)
    bad = _teacher_dict()
    bad["pooled"] = torch.rand(1, L, 5, QB, QB)
    path3 = tmp_path / "bad.pt"
    torch.save(bad, path3)
    with pytest.raises(AssertionError, match="H=5 not divisible by G=2"):
        load_teacher(path3)


class _Payload:
    pass


def test_pickled_objects_are_refused(tmp_path):
    d = _teacher_dict()
    d["extra"] = _Payload()
    path = tmp_path / "obj.pt"
    torch.save(d, path)
    with pytest.raises(Exception, match="[Ww]eights only load failed|Unsupported global"):
        load_selector_features(path)


def test_causal_block_mask():
    m = causal_block_mask(3, 4)
    assert m.tolist() == [[True, False, False, False], [True, True, False, False], [True, True, True, False]]
