"""The split policy of quantized.rs as pure logic (no GPU): which tensors are
quantized, at how many bits, and which stay dense."""
from __future__ import annotations

from sdq import quantized as q


def test_constants():
    assert q.GROUP_SIZE == 64 and q.DEFAULT_BITS == 4  # quantized.rs:45-49


def test_quantizable_is_two_d_with_a_divisible_width():
    # quantized.rs:172-174; mlx_quantized.rs:148-179 exercises the same cases.
    assert q.quantizable([128, 256])
    assert not q.quantizable([128])          # a bias or a norm
    assert not q.quantizable([32, 100])      # 100 does not divide by 64
    assert not q.quantizable([2, 3, 64])     # not 2-D


def test_sensitive_names_get_eight_bits():
    policy = q.mixed(4)
    for name in ("double_blocks.0.img_mod.lin.weight", "single_blocks.3.modulation.lin.weight",
                 "time_embedder.linear_1.weight", "img_in.weight", "txt_in.weight",
                 "final_layer.linear.weight", "final_layer.adaLN_modulation.1.weight"):
        assert q.sensitive(name)
        assert policy(name) == 8, name


def test_indexed_names_stay_dense():
    policy = q.mixed(4)
    for name in ("shared.weight", "encoder.block.0.layer.0.SelfAttention.relative_attention_bias.weight",
                 "pos_embed", "x_embedder.proj.weight", "model.embed_tokens.weight", "lm_head.weight"):
        assert q.indexed(name)
        assert policy(name) == 0, name


def test_everything_else_takes_the_requested_bits():
    # Under the reference's mixed(4), residual writers (attn.proj, mlp.2,
    # linear2) stay at 4 bits; the BASELINE configs use 8 for them instead.
    for bits in (4, 8):
        policy = q.mixed(bits)
        for name in ("double_blocks.0.img_attn.qkv.weight", "double_blocks.0.img_attn.proj.weight",
                     "double_blocks.0.img_mlp.0.weight", "double_blocks.0.img_mlp.2.weight",
                     "single_blocks.0.linear1.weight", "single_blocks.0.linear2.weight",
                     "time_in.in_layer.weight", "vector_in.out_layer.weight"):
            assert policy(name) == bits, name
