"""ixh_model_load_safetensors: an indecis model.safetensors (the layout
Save writes, model.go:494-560) loaded straight into device memory gives
the encoder the oracle computes from the same float weights (PackB8 of
each matrix, the table in its stored format), bit for bit."""
import numpy as np
import pytest

from helpers import f32_bits_equal, ids_uniform_lengths, mismatch_report, small_cfg
from indecis_amd import _lib
from indecis_amd import safetensors as st
from indecis_amd.modernbert import EMB_BF16, EMB_F32, EMB_I8, Model, Weights
from oracle import oracle as orc

pytestmark = pytest.mark.gpu


def _float_model(cfg, seed):
    """Float32 weights (matrices N(0, 0.03), norms U(0.9, 1.1), table
    N(0, 1)) and the Weights the oracle runs on: each matrix through the
    oracle's PackB8 (int8.go:38-77)."""
    rng = np.random.default_rng(seed)
    H, I, L, V = cfg.hidden, cfg.intermediate, cfg.layers, cfg.vocab
    f = {"emb": rng.standard_normal((V, H), dtype=np.float32),
         "emb_norm": rng.uniform(0.9, 1.1, H).astype(np.float32),
         "final_norm": rng.uniform(0.9, 1.1, H).astype(np.float32), "layers": []}
    for _ in range(L):
        f["layers"].append({
            "qkv": (rng.standard_normal((3 * H, H)) * 0.03).astype(np.float32),
            "o": (rng.standard_normal((H, H)) * 0.03).astype(np.float32),
            "i": (rng.standard_normal((2 * I, H)) * 0.03).astype(np.float32),
            "omlp": (rng.standard_normal((H, I)) * 0.03).astype(np.float32),
            "attn_norm": rng.uniform(0.9, 1.1, H).astype(np.float32),
            "mlp_norm": rng.uniform(0.9, 1.1, H).astype(np.float32)})
    w = Weights(cfg)
    for key, n, k in (("qkv", 3 * H, H), ("o", H, H), ("i", 2 * I, H), ("omlp", H, I)):
        qs = [orc.pack_b8(f["layers"][l][key], k, n) for l in range(L)]
        setattr(w, {"qkv": "wqkv", "o": "wo", "i": "wi", "omlp": "womlp"}[key] + "_q", np.stack([q for q, _, _ in qs]))
        setattr(w, {"qkv": "wqkv", "o": "wo", "i": "wi", "omlp": "womlp"}[key] + "_s", np.stack([s for _, s, _ in qs]))
    w.attn_norm = np.stack([f["layers"][l]["attn_norm"] for l in range(L)])
    w.mlp_norm = np.stack([f["layers"][l]["mlp_norm"] for l in range(L)])
    w.emb_norm, w.final_norm = f["emb_norm"], f["final_norm"]
    return f, w


def _save(path, cfg, f, w, emb_format, prefix="", mat_dtype="F32"):
    """Save (model.go:494-560): the table as bf16 + the exact rows, or int8
    + per-row scales; matrices and norms in F32 (or BF16 when exactly
    representable)."""
    t = {}
    if emb_format == EMB_BF16:
        t[prefix + "embeddings.tok_embeddings.weight"] = (
            (w.emb_bf16.astype(np.uint32) << 16).view(np.float32).reshape(cfg.vocab, cfg.hidden), "BF16")
        t["indecis.embeddings.exact_rows"] = w.emb_exact_ids.astype(np.float32)
        t["indecis.embeddings.exact_values"] = w.emb_exact_rows
    elif emb_format == EMB_I8:
        t[prefix + "embeddings.tok_embeddings.weight"] = (w.emb_i8.astype(np.float32), "I8")
        t["indecis.embeddings.scale"] = w.emb_i8_scale
    else:
        t[prefix + "embeddings.tok_embeddings.weight"] = w.emb_f32
    t[prefix + "embeddings.norm.weight"] = f["emb_norm"]
    t[prefix + "final_norm.weight"] = f["final_norm"]
    for l, lay in enumerate(f["layers"]):
        p = f"{prefix}layers.{l}."
        if l > 0:
            t[p + "attn_norm.weight"] = lay["attn_norm"]
        t[p + "mlp_norm.weight"] = lay["mlp_norm"]
        for key, name in (("qkv", "attn.Wqkv.weight"), ("o", "attn.Wo.weight"), ("i", "mlp.Wi.weight"),
                          ("omlp", "mlp.Wo.weight")):
            t[p + name] = (lay[key], mat_dtype)
    st.write(path, t, {"format": "indecis"})


@pytest.mark.parametrize("emb_format,prefix,mat_dtype", [
    (EMB_BF16, "", "F32"), (EMB_I8, "model.", "F32"), (EMB_F32, "", "BF16")])
def test_load_equals_oracle(tmp_path, emb_format, prefix, mat_dtype):
    cfg = small_cfg(layers=3)
    f, w = _float_model(cfg, seed=40)
    if mat_dtype == "BF16":
        # bf16-exact matrices, as Save writes an untrained backbone: the
        # oracle packs the same (rounded) floats
        for lay in f["layers"]:
            for key in ("qkv", "o", "i", "omlp"):
                lay[key] = (st.to_bf16(lay[key]).astype(np.uint32) << 16).view(np.float32).reshape(lay[key].shape)
        f, w = f, _float_model_from(cfg, f)
    w.set_embeddings(f["emb"], emb_format, rng=np.random.default_rng(41))
    path = tmp_path / "model.safetensors"
    _save(path, cfg, f, w, emb_format, prefix, mat_dtype)
    gpu = Model.open(cfg, path, lanes=8)
    ora = orc.OracleModel(w, lanes=8)
    rng = np.random.default_rng(42)
    seqs = ids_uniform_lengths(rng, 6, 1, 200, cfg.vocab)
    got = gpu.encode_seqs(seqs)
    want = ora.encode_seqs(seqs)
    gpu.close()
    assert f32_bits_equal(got, want), mismatch_report(got, want)


def _float_model_from(cfg, f):
    """Weights for the oracle from float matrices already fixed in f."""
    H, I, L = cfg.hidden, cfg.intermediate, cfg.layers
    w = Weights(cfg)
    for key, attr, n, k in (("qkv", "wqkv", 3 * H, H), ("o", "wo", H, H), ("i", "wi", 2 * I, H),
                            ("omlp", "womlp", H, I)):
        qs = [orc.pack_b8(f["layers"][l][key], k, n) for l in range(L)]
        setattr(w, attr + "_q", np.stack([q for q, _, _ in qs]))
        setattr(w, attr + "_s", np.stack([s for _, s, _ in qs]))
    w.attn_norm = np.stack([f["layers"][l]["attn_norm"] for l in range(L)])
    w.mlp_norm = np.stack([f["layers"][l]["mlp_norm"] for l in range(L)])
    w.emb_norm, w.final_norm = f["emb_norm"], f["final_norm"]
    return w


def test_load_errors(tmp_path):
    """A missing tensor, a wrong shape, an int8 table without scales and a
    corrupt file give the reference's messages."""
    cfg = small_cfg(layers=2)
    f, w = _float_model(cfg, seed=43)
    w.set_embeddings(f["emb"], EMB_F32)
    path = tmp_path / "m.safetensors"
    _save(path, cfg, f, w, EMB_F32)
    bad = small_cfg(layers=3)
    with pytest.raises(_lib.IxhError, match="modernbert: tensor layers.2.attn_norm.weight missing"):
        Model.open(bad, path)
    f["layers"][1]["o"] = f["layers"][1]["o"][:, :-1].copy()
    _save(path, cfg, f, w, EMB_F32)
    with pytest.raises(_lib.IxhError, match=r"layers.1.attn.Wo.weight: shape \[256 255\], expected \[256 256\]"):
        Model.open(cfg, path)
    w.set_embeddings(f["emb"], EMB_I8)
    f["layers"][1]["o"] = f["layers"][1]["o"]
    t_path = tmp_path / "noscale.safetensors"
    st.write(t_path, {"embeddings.tok_embeddings.weight": (w.emb_i8.astype(np.float32), "I8")})
    with pytest.raises(_lib.IxhError, match="indecis: int8 table without scales"):
        Model.open(cfg, t_path)
    (tmp_path / "short").write_bytes(b"\x01\x02")
    with pytest.raises(_lib.IxhError, match="safetensors: truncated file"):
        Model.open(cfg, tmp_path / "short")
