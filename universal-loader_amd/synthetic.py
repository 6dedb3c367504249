"""Random-init Llama-shaped models synthesized on the device (no checkpoint is
loaded): every linear tensor and the embedding are N(0, std^2) values from the
counter-based stream (seed, i) quantized to GGUF blocks by ulspec_synth_q4;
norm weights are 1.  Tensor names follow the GGUF weight map of
Model::load_from_gguf (src/inference/model.cpp:190-246)."""
import collections

import numpy as np

DeviceSpan = collections.namedtuple("DeviceSpan", "ptr nbytes")


def tensor_shapes(dim, n_layers, n_heads, n_kv_heads, ffn, vocab, **_):
    """(name, ne0, ne1) of every quantized tensor; the list index is the
    synthesis stream of the tensor."""
    D = dim // n_heads
    out = [("token_embd.weight", dim, vocab), ("output.weight", dim, vocab)]
    for l in range(n_layers):
        out += [(f"blk.{l}.attn_q.weight", dim, n_heads * D), (f"blk.{l}.attn_k.weight", dim, n_kv_heads * D),
                (f"blk.{l}.attn_v.weight", dim, n_kv_heads * D), (f"blk.{l}.attn_output.weight", n_heads * D, dim),
                (f"blk.{l}.ffn_gate.weight", dim, ffn), (f"blk.{l}.ffn_up.weight", dim, ffn),
                (f"blk.{l}.ffn_down.weight", ffn, dim)]
    return out


def norm_names(n_layers, **_):
    return ["output_norm.weight"] + [f"blk.{l}.{n}.weight" for l in range(n_layers) for n in ("attn_norm", "ffn_norm")]


def synthetic_llama(pkg, ctx, cfg, wtype, seed, std=0.02, keep_host=False):
    """Create a Model with synthetic weights.  With keep_host, also return the
    raw GGUF bytes of every tensor as {name: (type, bytes, ne0, ne1)}."""
    cfg = dict(cfg)
    n_seq = cfg.pop("n_seq", 1)
    model = pkg.Model(ctx, **cfg, n_seq=n_seq)
    shapes = tensor_shapes(**cfg)
    biggest = max(ne1 * pkg.row_bytes(wtype, ne0) for _, ne0, ne1 in shapes)
    buf = ctx.alloc(biggest)
    host = {} if keep_host else None
    try:
        for i, (name, ne0, ne1) in enumerate(shapes):
            nbytes = ne1 * pkg.row_bytes(wtype, ne0)
            ctx.synth_q4(wtype, seed, i, ne1, ne0, std, buf)
            model.set_tensor(name, wtype, DeviceSpan(buf.ptr, nbytes), ne0, ne1)
            if keep_host:
                host[name] = (wtype, ctx.download(buf, np.uint8, (nbytes,)), ne0, ne1)
    finally:
        buf.free()
    ones = np.ones(cfg["dim"], np.float32)
    for name in norm_names(**cfg):
        model.set_tensor(name, 0, ones, cfg["dim"], 1)
        if keep_host:
            host[name] = (0, ones, cfg["dim"], 1)
    return model, host
