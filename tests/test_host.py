"""Host-side logic of the drop-in modules (CPU only, no kernel launches)."""
import pytest
import torch

from oracle import swin_oracle as so
from terra_amd import kernels, utils
from terra_amd.attention import WindowAttention, relative_position_index
from terra_amd.kernels import ShiftMask, WindowGeometry
from terra_amd.transformer import SequentialSwinTransformer
from terra_amd.workloads import CONFIGS


@pytest.mark.parametrize("H,W,ws,s", [(56, 56, 7, 3), (16, 24, 8, 4), (32, 64, 8, 4), (24, 16, 8, 2)])
def test_dense_mask_equals_oracle(H, W, ws, s):
    assert torch.equal(utils.get_swin_attention_mask("sequential", (H, W), ws, s), so.shift_mask(H, W, ws, s))


def test_dense_mask_parallel_mode_is_out_of_scope():
    with pytest.raises(NotImplementedError):
        utils.get_swin_attention_mask("parallel", (16, 16), 8, 4)


@pytest.mark.parametrize("ws", [(7, 7), (8, 8), (6, 6), (4, 7)])
def test_relative_index_closed_form_equals_oracle(ws):
    assert torch.equal(relative_position_index(ws), so.relative_position_index(ws))


@pytest.mark.parametrize("res,win,want", [
    ((2, 721, 1440), (2, 8, 8), (0, 0, 3, 4, 0, 0)),
    ((3, 720, 1443), (2, 8, 8), (2, 3, 0, 0, 0, 1)),
    ((4, 64, 64), (2, 8, 8), (0, 0, 0, 0, 0, 0)),
])
def test_get_pad3d(res, win, want):
    assert utils.get_pad3d(res, win) == want


def test_get_pad2d():
    assert utils.get_pad2d((721, 1443), (8, 8)) == (2, 3, 3, 4)


def test_pack_key_bits():
    flags = torch.zeros(3, 64, dtype=torch.bool)
    flags[0, 0] = True
    flags[1, 63] = True
    flags[2, 5] = flags[2, 7] = True
    bits = utils.pack_key_bits(flags)
    assert bits.tolist() == [1, -(1 << 63), (1 << 5) | (1 << 7)]


def test_geometry_and_shift_mask_descriptor():
    cfg = CONFIGS["c5"]
    g = WindowGeometry(cfg.batch, cfg.height, cfg.width, cfg.channels, cfg.window, 4, 4, cfg.pad,
                       cfg.win_row_begin, cfg.win_rows, cfg.valid)
    assert (g.frame_h, g.frame_w, g.rows, g.cols) == (304, 512, 37, 64)
    assert g.num_windows == 4736 == cfg.num_windows
    m = ShiftMask.from_geometry(g)
    assert (m.frame_h, m.frame_w, m.win_rows, m.win_cols) == (304, 512, 37, 64)
    c = g.to_c()
    assert (c.valid_begin, c.valid_end, c.pad_bottom, c.win_rows) == (27, 2358, 8, 37)


def test_config_sizes():
    assert CONFIGS["c3"].num_windows == 8192 and CONFIGS["c3"].tokens == 64
    assert CONFIGS["c2"].num_windows == 1024 and CONFIGS["c1"].num_windows == 64
    assert CONFIGS["c4"].num_windows == 512
    assert CONFIGS["c5"].real_tokens == 2 * 2331 * 64


REFERENCE_KEYS = [
    "norm1.weight", "norm1.bias",
    "attn.relative_position_bias_table", "attn.relative_position_index",
    "attn.q_linear.weight", "attn.q_linear.bias", "attn.k_linear.weight", "attn.k_linear.bias",
    "attn.v_linear.weight", "attn.v_linear.bias", "attn.proj.weight", "attn.proj.bias",
]


def test_block_state_dict_keys_match_reference():
    blk = SequentialSwinTransformer(layer_idx=1, height=16, width=16, embedding_dim=64, window_size=8,
                                    num_heads=2)
    # own buffers precede submodules in a state dict, as in the reference module
    assert list(blk.state_dict().keys()) == ["attn_mask"] + REFERENCE_KEYS
    assert blk.shift_size == 4
    assert torch.equal(blk.attn_mask, so.shift_mask(16, 16, 8, 4))
    blk0 = SequentialSwinTransformer(layer_idx=0, height=16, width=16, embedding_dim=64, window_size=8,
                                     num_heads=2)
    assert list(blk0.state_dict().keys()) == REFERENCE_KEYS
    assert blk0.shift_size == 0 and blk0.attn_mask is None
    # a reference-layout state dict (same names, shapes) loads strictly
    sd = {k: torch.randn_like(v.float()).to(v.dtype) if v.is_floating_point() else v
          for k, v in blk.state_dict().items()}
    blk.load_state_dict(sd, strict=True)
    assert torch.equal(blk.attn.proj.weight, sd["attn.proj.weight"])


def test_window_attention_init_is_seeded_and_restores_rng():
    torch.manual_seed(5)
    before = torch.rand(1)
    torch.manual_seed(5)
    a = WindowAttention(64, (8, 8), 2, init_seed_base=123)
    after = torch.rand(1)
    assert torch.equal(before, after)  # global RNG untouched by seeded init
    b = WindowAttention(64, (8, 8), 2, init_seed_base=123)
    for (ka, va), (kb, vb) in zip(a.state_dict().items(), b.state_dict().items()):
        assert ka == kb and torch.equal(va, vb)
    # trunc_normal_(std=.02) with the default absolute bounds [-2, 2]
    t = a.relative_position_bias_table.detach()
    assert 0.015 < float(t.std()) < 0.025 and float(t.abs().max()) <= 2.0
    assert a.scale == 32 ** -0.5


def test_window_mask_descriptor_of_block():
    blk = SequentialSwinTransformer(layer_idx=1, height=16, width=24, embedding_dim=64, window_size=8,
                                    num_heads=2)
    m = blk.window_mask(blk.geometry(2))
    assert isinstance(m.shift, ShiftMask) and m.land_bits is None
    assert (m.shift.frame_h, m.shift.frame_w, m.shift.shift_h, m.shift.win_rows, m.shift.win_cols) == (16, 24, 4, 2, 3)
    blk0 = SequentialSwinTransformer(layer_idx=0, height=16, width=24, embedding_dim=64, window_size=8,
                                     num_heads=2)
    assert blk0.window_mask(blk0.geometry(1)) is None


def test_mlp_workload_is_seeded_and_named_like_the_reference():
    from terra_amd import workloads
    cfg = workloads.CONFIGS["c3"]
    a, b = workloads.mlp_for(cfg, 1), workloads.mlp_for(cfg, 1)
    assert sorted(a.state_dict()) == ["fc1.bias", "fc1.weight", "fc2.bias", "fc2.weight", "norm2.bias",
                                      "norm2.weight"]
    assert a.fc1.weight.shape == (4 * cfg.channels, cfg.channels)
    assert all(torch.equal(a.state_dict()[k], b.state_dict()[k]) for k in a.state_dict())
    assert not torch.equal(a.fc1.weight, workloads.mlp_for(cfg, 0).fc1.weight)


def test_window_mask_land_bits_follow_the_frame(monkeypatch):
    """The block's cached land bits are rebuilt when the frame changes (here
    the emitted window rows) even though the land grid is the same tensor."""
    import terra_amd.transformer as tr

    seen = []

    def fake_bits(land, geom):  # host stand-in for the HIP gather: records the frame it was asked for
        seen.append(geom.win_row_begin)
        return torch.tensor([geom.win_row_begin, geom.rows], dtype=torch.int64)

    monkeypatch.setattr(tr, "land_window_bits", fake_bits)
    land = torch.zeros(32, 16, dtype=torch.bool)
    blk = SequentialSwinTransformer(layer_idx=1, height=32, width=16, embedding_dim=16, window_size=8, num_heads=2,
                                    land_mask=land, win_row_begin=0, win_rows=2)
    m0 = blk.window_mask(blk.geometry(1))
    assert m0.land_bits.tolist() == [0, 2]
    assert blk.window_mask(blk.geometry(1)) is m0  # unchanged frame: cached
    blk.win_row_begin = 1
    m1 = blk.window_mask(blk.geometry(1))
    assert m1.land_bits.tolist() == [1, 2]
    assert seen == [0, 1]
