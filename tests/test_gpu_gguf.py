"""GGUF file -> HBM on the GPU: a written qwen3moe file (mixed Q4_0 / Q4_1 / Q6_K down, split
into shards) loaded with qmsg_gguf_upload must hold the file's bytes, and the layers and the
chain over them must reproduce the oracle bit for bit."""
import numpy as np
import pytest

import gguf_file as gf
import oracle as orc

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def q():
    from large_model_amd import qmsg
    return qmsg


def layers(E, X, K, F, types, seed=60):
    return [orc.Layer(E, X, K, F, seed + l, layer=l, down_type=dt) for l, dt in enumerate(types)]


@pytest.mark.parametrize("shards", [1, 2])
def test_gguf_layers_and_chain_exact(q, tmp_path, shards):
    E, X, K, F, T = 512, 16, 4, 256, 5
    lays = layers(E, X, K, F, (orc.T_Q4_0, orc.T_Q4_1, orc.T_Q6_K))
    path, norms = gf.moe_model(str(tmp_path / "m.gguf"), lays, eps=1e-6, n_shards=shards)
    print(f"[case] gguf shards={shards} E={E} X={X} K={K} F={F} T={T}", flush=True)
    x = orc.make_input(E, T, 3)
    h0 = orc.make_input(E, T, 4) * np.float32(3.0)
    with q.Gguf(path) as g, q.Context.from_gguf(g, max_tokens=T) as ctx:
        assert (ctx.E, ctx.X, ctx.K, ctx.F, ctx.n_layer) == (E, X, K, F, 3)
        for l, lay in enumerate(lays):
            r, gate, up, down = ctx.download(l)
            assert np.array_equal(r, lay.router) and np.array_equal(gate, lay.gate), l
            assert np.array_equal(up, lay.up) and np.array_equal(down, lay.down), l
            out = ctx.moe(l, x)
            assert np.array_equal(out.view(np.uint32), lay.moe(x).view(np.uint32)), l
        # the MoE half of the layer loop with the file's ffn_norm weights and eps
        h = h0.copy()
        for l, lay in enumerate(lays):
            h = h + lay.moe(orc.rmsnorm(h, norms[l], eps=ctx.eps))
        d_h = ctx.device_alloc(h0.nbytes)
        ctx.h2d(d_h, h0)
        ctx.moe_chain(0, 3, d_h, T, eps=ctx.eps)
        ctx.sync()
        got = ctx.d2h(d_h, (T, E))
    assert np.array_equal(got.view(np.uint32), h.view(np.uint32))


def test_gguf_upload_checks_shapes_and_range(q, tmp_path):
    E, X, K, F = 256, 16, 4, 128
    lays = layers(E, X, K, F, (orc.T_Q4_0, orc.T_Q4_0))
    path, _ = gf.moe_model(str(tmp_path / "m.gguf"), lays)
    # a file whose layer 1 down tensor has the wrong expert count
    bad = str(tmp_path / "bad.gguf")
    with q.Gguf(path) as g:
        tabs = g.tensors()
    raw = open(path, "rb").read()
    ts = []
    for t in tabs:
        ne = t["ne"][:t["n_dims"]]
        if t["name"] == "blk.1.ffn_down_exps.weight":
            ne = [ne[0], ne[1], ne[2] // 2]
        data = raw[t["off"]:t["off"] + t["nbytes"]]
        ts.append((t["name"], t["type"], ne, data[:len(data) // 2] if ne != t["ne"][:t["n_dims"]] else data))
    with q.Gguf(path) as g:
        kvs = [("general.architecture", gf.STR, "qwen3moe")] + [
            (k, gf.U32, g.get_int(k)) for k in ("qwen3moe.block_count", "qwen3moe.embedding_length",
                                                 "qwen3moe.expert_count", "qwen3moe.expert_used_count",
                                                 "qwen3moe.expert_feed_forward_length")] + [
            ("qwen3moe.attention.layer_norm_rms_epsilon", gf.F32, 1e-6)]
    gf.write_gguf(bad, kvs, ts)
    x = orc.make_input(E, 2, 1)
    with q.Gguf(bad) as g, q.Context(E, X, K, F, n_layer=2, max_tokens=2) as ctx:
        ctx.load_gguf(g, 0, 1)                   # layer 0 is intact
        assert np.array_equal(ctx.moe(0, x).view(np.uint32), lays[0].moe(x).view(np.uint32))
        with pytest.raises(q.QmsgError, match="ffn_down_exps") as ei:
            ctx.load_gguf(g, 1, 1)
        assert ei.value.status == -1
        with pytest.raises(q.QmsgError) as ei:
            ctx.load_gguf(g, 1, 2)               # layers 1..2 of a 2-layer context
        assert ei.value.status == -5
        with pytest.raises(q.QmsgError):
            ctx.moe(1, x)                        # layer 1 never got weights
    with q.Gguf(path) as g, q.Context(E, X, K, F + 64, n_layer=2, max_tokens=2) as ctx:
        with pytest.raises(q.QmsgError):
            ctx.load_gguf(g, 0, 1)               # the file's n_ff_exp differs from the context's


def test_gguf_q8_0_f16_experts_off_grid(q, tmp_path):
    """A written file with Q8_0 and F16 / F32 expert tensors (Q8_0 GGUF files carry them) at an
    n_embd off the integer kernels' grid: loaded, bit for bit per layer and over the chain."""
    import expert_types as et
    E, X, K, F, T = 288, 12, 3, 160, 4
    lays = [et.typed_layer(E, X, K, F, types, 70 + 10 * l)
            for l, types in enumerate(((orc.T_Q8_0, orc.T_Q8_0, orc.T_Q8_0),
                                       (orc.T_F16, orc.T_Q8_0, orc.T_F32)))]
    path, norms = gf.moe_model(str(tmp_path / "q8.gguf"), lays, eps=1e-6)
    print(f"[case] gguf q8_0/f16 E={E} F={F} T={T}", flush=True)
    x = orc.make_input(E, T, 5, rmsnorm=True)
    h0 = orc.make_input(E, T, 6) * np.float32(3.0)
    with q.Gguf(path) as g, q.Context.from_gguf(g, max_tokens=T) as ctx:
        for l, lay in enumerate(lays):
            r, gate, up, down = ctx.download(l)
            assert np.array_equal(gate, lay.gate) and np.array_equal(up, lay.up) and np.array_equal(down, lay.down)
            assert np.array_equal(ctx.moe(l, x).view(np.uint32), lay.moe(x).view(np.uint32)), l
        h = h0.copy()
        for l, lay in enumerate(lays):
            h = h + lay.moe(orc.rmsnorm(h, norms[l], eps=ctx.eps))
        d_h = ctx.device_alloc(h0.nbytes)
        ctx.h2d(d_h, h0)
        ctx.moe_chain(0, 2, d_h, T, eps=ctx.eps)
        ctx.sync()
        got = ctx.d2h(d_h, (T, E))
    assert np.array_equal(got.view(np.uint32), h.view(np.uint32))
