"""Models read from GGUF files (ulspec_model_load_gguf) on the GPU: the same
bytes through the file give bitwise the same logits and speculative loop as
through ulspec_model_set_tensor, and the logits stay within the tolerance of
test_spec_gpu.py of the oracle model built from the same tensors."""
import numpy as np
import pytest

import gguf_io as G
from llama_util import load, make_tensors

pytestmark = pytest.mark.gpu

CFG = dict(dim=256, n_layers=2, n_heads=4, n_kv_heads=2, ffn=512, vocab=1000, max_ctx=64, rms_eps=1e-5,
           rope_base=10000.0)


@pytest.fixture(scope="module", params=[2, 12], ids=["q4_0", "q4_k"])
def model_file(request, ora, tmp_path_factory):
    wtype = request.param
    t = make_tensors(ora, CFG, wtype, seed=5 + wtype, norm_std=0.1)
    p = tmp_path_factory.mktemp("gguf") / f"tiny_{wtype}.gguf"
    G.write(p, G.llama_kv(CFG), G.model_tensors(t))
    return p, t


def test_file_model_equals_set_tensor_model(pkg, ctx, ora, model_file):
    path, tensors = model_file
    print(f"  loading {path.name}", flush=True)
    fm = pkg.load_gguf_model(ctx, str(path))
    assert (fm.cfg.dim, fm.cfg.n_layers, fm.cfg.vocab, fm.cfg.max_ctx) == (256, 2, 1000, 64)
    sm = pkg.Model(ctx, **CFG)
    load(sm, tensors)
    toks = np.random.default_rng(3).integers(0, CFG["vocab"], 12).astype(np.int32)
    lf, ls = fm.forward(toks, 0, n_logits=12), sm.forward(toks, 0, n_logits=12)
    assert np.array_equal(lf.view(np.uint32), ls.view(np.uint32))
    om = ora.Llama(**CFG, nthreads=ora.nthreads_default())
    load(om, tensors)
    lo = om.forward(toks, 0, n_logits=12)
    err = np.abs(lf.astype(np.float64) - lo).max() / np.sqrt((lo.astype(np.float64) ** 2).mean())
    print(f"  logits max err / rms vs oracle = {err:.2e}")
    assert err <= 1e-2
    fm.close()
    sm.close()


def test_speculative_loop_from_files(pkg, ctx, model_file):
    """Target and draft from GGUF files: the greedy loop commits the same
    tokens as with the models built tensor by tensor."""
    path, tensors = model_file
    prompt = np.random.default_rng(9).integers(0, CFG["vocab"], 16).astype(np.int32)
    out = []
    for from_file in (True, False):
        if from_file:
            t, d = pkg.load_gguf_model(ctx, str(path)), pkg.load_gguf_model(ctx, str(path))
        else:
            t, d = pkg.Model(ctx, **CFG), pkg.Model(ctx, **CFG)
            load(t, tensors)
            load(d, tensors)
        sp = pkg.Speculative(t, d, 3, pkg.sampling(greedy=True), 11)
        sp.prefill(prompt)
        sp.generate(24)
        out.append(sp.tokens())
        sp.close()
        t.close()
        d.close()
    assert np.array_equal(out[0], out[1])


def test_unsupported_tensor_type_is_named(pkg, ctx, model_file, tmp_path):
    path, tensors = model_file
    tens = G.model_tensors(tensors)
    ne = (CFG["dim"], CFG["vocab"])
    # Q5_K (13, 176 B per 256) is a GGUF type the kernels do not read
    tens = [x if x[0] != "output.weight" else ("output.weight", 13, ne, bytes(G.tensor_nbytes(13, ne)))
            for x in tens]
    p = tmp_path / "q5k.gguf"
    G.write(p, G.llama_kv(CFG), tens)
    with pytest.raises(pkg.UlspecError, match="output.weight") as e:
        pkg.load_gguf_model(ctx, str(p))
    assert e.value.status == pkg.EUNSUPPORTED
