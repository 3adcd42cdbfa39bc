"""Helpers shared by the decoder tests: build the oracle decoder and the synthetic models."""
import numpy as np

from conftest import load_package

LAYER_ORDER = ("input_layernorm.weight", "self_attn.q_proj.weight", "self_attn.k_proj.weight", "self_attn.v_proj.weight",
               "self_attn.o_proj.weight", "self_attn.q_proj.bias", "self_attn.k_proj.bias", "self_attn.v_proj.bias",
               "post_attention_layernorm.weight", "mlp.gate_proj.weight", "mlp.up_proj.weight",
               "mlp.down_proj.weight")


def qnt_module():
    load_package()
    import quanta_cpp_amd.qnt as qnt
    return qnt


def hp_dict(hp, ctx_len=None):
    return dict(vocab=hp.vocab_size, dim=hp.dim, n_layers=hp.n_layers, n_heads=hp.n_heads, n_kv_heads=hp.n_kv_heads,
                head_dim=hp.head_dim, ffn_dim=hp.ffn_dim, ctx_len=ctx_len or hp.max_seq, qkv_bias=int(hp.qkv_bias),
                rope_theta=hp.rope_theta, norm_eps=hp.norm_eps)


def oracle_decoder(oracle, hp, tensors, ctx_len=None):
    arrays, dtypes = [], []

    def add(name):
        t = tensors.get(name)
        arrays.append(None if t is None else np.asarray(t.data))
        dtypes.append(-1 if t is None else t.dtype)

    add("model.embed_tokens.weight")
    add("model.norm.weight")
    for l in range(hp.n_layers):
        for n in LAYER_ORDER:
            add(f"model.layers.{l}.{n}")
    add("quanta.head_q4")
    add("quanta.head_err")
    return oracle.decoder(hp_dict(hp, ctx_len), arrays, dtypes)
