"""Shared model set-up for the decode tests: dims, host tensors of the
random-init model (same bytes the GPU model is built from)."""
import arcllm_amd as arc


def tiny_dims(layers=3, vocab=4096):
    d = arc.ModelDims()
    d.hidden, d.q_heads, d.kv_heads, d.head_dim = 512, 4, 2, 128
    d.ffn, d.vocab, d.layers = 1024, vocab, layers
    d.rms_eps, d.rope_theta = 1e-6, 1e6
    for layer in range(layers):  # mix both quantisations of attn_v and ffn_down
        d.v_type[layer] = arc.Q4_K if layer % 3 == 0 else arc.Q6_K
        d.down_type[layer] = arc.Q4_K if layer % 3 == 1 else arc.Q6_K
    return d
