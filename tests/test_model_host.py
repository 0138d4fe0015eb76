"""Host-side checks of the decoder-stack driver (crane_amd/model.py) that
need no GPU: the CLA anchor map of Hunyuan's cross-layer attention
(hunyuan_dense/modeling.rs:1035-1059: layer i with i % f != 0 reuses layer
i - i % f's K/V), weight-shape validation, and that a step on CPU tensors
is rejected (there is no CPU fallback)."""
import pytest
import torch

from crane_amd import CraneHipError, decoder, model

D = 128


def _layers(cfg, shared_rows=None):
    H, Hq, Hkv, I = cfg.hidden, cfg.num_heads, cfg.num_kv_heads, cfg.intermediate
    out = []
    for i in range(cfg.num_layers):
        shared = cfg.cla_share_factor > 1 and i % cfg.cla_share_factor != 0
        rows = (Hq if shared else Hq + 2 * Hkv) * D
        if shared_rows is not None and shared:
            rows = shared_rows
        z = lambda *s: torch.zeros(s, dtype=torch.bfloat16)
        out.append(decoder.LayerWeights(input_norm=z(H), qkv=z(rows, H), o=z(H, Hq * D), post_norm=z(H),
                                        gate_up=z(2 * I, H), down=z(H, I)))
    return out


def test_cla_anchor_map_and_caches():
    cfg = model.ModelConfig(hidden=256, num_heads=4, num_kv_heads=2, intermediate=512, num_layers=6,
                            family="hunyuan", rope_theta=1e4, rope_alpha=1000.0, max_position=64,
                            cla_share_factor=3)
    m = model.DecoderModel(cfg, _layers(cfg), torch.zeros(256, dtype=torch.bfloat16), None, 2, 16)
    assert [m.shared(i) for i in range(6)] == [False, True, True, False, True, True]
    assert [m.anchor(i) for i in range(6)] == [0, 0, 0, 3, 3, 3]
    assert [k is None for k in m.k] == [False, True, True, False, True, True]   # shared layers keep no cache
    assert m.k[0].shape == (2, 2, 16, D)


def test_bad_shapes_and_cpu_step_are_rejected():
    cfg = model.ModelConfig(hidden=256, num_heads=4, num_kv_heads=2, intermediate=512, num_layers=2,
                            cla_share_factor=2, family="hunyuan")
    with pytest.raises(CraneHipError):     # a CLA shared layer must carry the q-only projection
        model.DecoderModel(cfg, _layers(cfg, shared_rows=8 * D), torch.zeros(256, dtype=torch.bfloat16), None, 1, 8)
    with pytest.raises(CraneHipError):
        model.DecoderModel(model.ModelConfig(256, 4, 2, 512, 2, family="llama"), _layers(cfg),
                           torch.zeros(256, dtype=torch.bfloat16), None, 1, 8)
    m = model.DecoderModel(cfg, _layers(cfg), torch.zeros(256, dtype=torch.bfloat16), None, 1, 8)
    x = torch.zeros((1, 2, 256), dtype=torch.bfloat16)
    with pytest.raises(CraneHipError, match="GPU only"):
        m.forward(x, torch.zeros(1, dtype=torch.int32))
    with pytest.raises(CraneHipError):     # past the capacity
        m.forward(torch.zeros((1, 9, 256), dtype=torch.bfloat16), torch.zeros(1, dtype=torch.int32))
