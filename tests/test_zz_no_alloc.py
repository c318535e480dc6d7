"""qmsg_moe_device_noalloc (the allocation-free layer call, scratch in the library's static
device array) against qmsg_moe_device on the same device buffers: bit for bit, on calls in a
row whose second input is smaller, on several shapes and paths, and its size limit; and the
same calls captured into a HIP graph and replayed."""
import ctypes

import numpy as np
import pytest

import oracle as orc

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def qmsg():
    from large_model_amd import qmsg as q
    return q


CASES = [
    # name, E, X, K, F, seed, token counts of the calls in a row, path
    ("q235b", 4096, 128, 8, 1536, 91, (16, 3, 1), "auto"),
    ("q235b_mfma", 4096, 128, 8, 1536, 92, (40, 5), "mfma"),
    ("q30b_t1", 2048, 128, 8, 768, 93, (1, 1), "auto"),
    ("tiny_fp32", 256, 16, 4, 128, 94, (7, 2), "fp32"),
]


@pytest.mark.parametrize("name,E,X,K,F,seed,Ts,path", CASES, ids=[c[0] for c in CASES])
def test_noalloc_equals_moe_device(qmsg, name, E, X, K, F, seed, Ts, path):
    print(f"[case] noalloc {name} T={Ts} path={path}", flush=True)
    Tm = max(Ts)
    with qmsg.Context(E, X, K, F, n_layer=1, max_tokens=Tm) as ctx:
        ctx.synth(0, seed)
        ctx.set_path({"auto": qmsg.PATH_AUTO, "mfma": qmsg.PATH_MFMA, "fp32": qmsg.PATH_FP32}[path])
        d_x = ctx.device_alloc(Tm * E * 4)
        d_ref = ctx.device_alloc(Tm * E * 4)
        d_got = ctx.device_alloc(Tm * E * 4)
        for i, T in enumerate(Ts):
            ctx.synth_input(seed + i, 0, T, d_x)
            ctx.moe_device(0, d_x, T, d_ref)
            ctx.moe_device_noalloc(0, d_x, T, d_got)
            ctx.sync()
            ref = ctx.d2h(d_ref, (T, E))
            got = ctx.d2h(d_got, (T, E))
            assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), (name, i, T)
            if name == "tiny_fp32":
                x = orc.make_input(E, T, seed + i)
                want = orc.Layer(E, X, K, F, seed).moe(x, exact=True)
                assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (name, i, "oracle")


def test_noalloc_limits(qmsg):
    """A batch whose scratch is above the static maximum is refused before any launch; T = 0 is a
    no-op; the context's max_tokens does not bound the call."""
    E, X, K, F = 4096, 128, 8, 1536
    with qmsg.Context(E, X, K, F, n_layer=1, max_tokens=1) as ctx:
        ctx.synth(0, 95)
        d_x = ctx.device_alloc(4 * E * 4)
        d_out = ctx.device_alloc(4 * E * 4)
        with pytest.raises(qmsg.QmsgError) as ei:
            ctx.moe_device_noalloc(0, d_x, 200, d_out)
        assert ei.value.status == -5 and "static maximum" in str(ei.value)
        ctx.moe_device_noalloc(0, d_x, 0, d_out)
        ctx.synth_input(95, 0, 4, d_x)
        ctx.moe_device_noalloc(0, d_x, 4, d_out)        # above max_tokens = 1
        ctx.sync()
        x = orc.make_input(E, 4, 95)
        want = orc.Layer(E, X, K, F, 95, experts=[]).moe(x)
        assert np.array_equal(ctx.d2h(d_out, (4, E)).view(np.uint32), want.view(np.uint32))


def test_noalloc_graph_replay(qmsg):
    """The calls the allocation-free entry point exists for: a sequence of layer calls (one token,
    then three, then one, on two layers) captured on the context's stream into a HIP graph and
    replayed three times. Between replays an eager call of another batch overwrites the shared
    static scratch and the outputs are cleared, so each replay must reset what it needs (the
    select launch's ticket counter, the record-range flags) itself. Every replay equals the
    eager run of the same calls bit for bit."""
    print("[case] noalloc graph replay", flush=True)
    hip = ctypes.CDLL("libamdhip64.so")
    vp = ctypes.c_void_p
    hip.hipStreamBeginCapture.argtypes = [vp, ctypes.c_int]
    hip.hipStreamEndCapture.argtypes = [vp, ctypes.POINTER(vp)]
    hip.hipGraphInstantiate.argtypes = [ctypes.POINTER(vp), vp, vp, vp, ctypes.c_size_t]
    hip.hipGraphLaunch.argtypes = [vp, vp]
    hip.hipStreamSynchronize.argtypes = [vp]
    hip.hipMemsetAsync.argtypes = [vp, ctypes.c_int, ctypes.c_size_t, vp]
    hip.hipGraphExecDestroy.argtypes = [vp]
    hip.hipGraphDestroy.argtypes = [vp]
    E, X, K, F, seed = 1024, 64, 8, 256, 97
    calls = [(0, 1), (1, 3), (0, 1)]            # (layer, tokens)
    row = E * 4
    with qmsg.Context(E, X, K, F, n_layer=2, max_tokens=4) as ctx:
        ctx.synth(0, seed)
        ctx.synth(1, seed + 1)
        st = vp(qmsg.lib.qmsg_stream(ctx._h))
        d_x = ctx.device_alloc(len(calls) * 4 * row)
        d_ref = ctx.device_alloc(len(calls) * 4 * row)
        d_got = ctx.device_alloc(len(calls) * 4 * row)
        for i, (_, T) in enumerate(calls):
            ctx.synth_input(seed + 10 + i, 0, T, d_x + i * 4 * row)
        d_other, d_other_out = ctx.device_alloc(4 * row), ctx.device_alloc(4 * row)
        ctx.synth_input(seed + 20, 0, 4, d_other)

        def run(dst):
            for i, (layer, T) in enumerate(calls):
                ctx.moe_device_noalloc(layer, d_x + i * 4 * row, T, dst + i * 4 * row)

        run(d_ref)
        ctx.sync()
        ref = [ctx.d2h(d_ref + i * 4 * row, (T, E)) for i, (_, T) in enumerate(calls)]
        graph, exe = vp(), vp()
        assert hip.hipStreamBeginCapture(st, 2) == 0          # relaxed capture mode
        run(d_got)
        assert hip.hipStreamEndCapture(st, ctypes.byref(graph)) == 0
        assert hip.hipGraphInstantiate(ctypes.byref(exe), graph, None, None, 0) == 0
        try:
            for rep in range(3):
                ctx.moe_device_noalloc(1, d_other, 4, d_other_out)  # eager work on the same scratch
                assert hip.hipMemsetAsync(vp(d_got), 0xff, len(calls) * 4 * row, st) == 0
                assert hip.hipGraphLaunch(exe, st) == 0
                assert hip.hipStreamSynchronize(st) == 0
                for i, (_, T) in enumerate(calls):
                    got = ctx.d2h(d_got + i * 4 * row, (T, E))
                    assert np.array_equal(got.view(np.uint32), ref[i].view(np.uint32)), (rep, i)
        finally:
            hip.hipGraphExecDestroy(exe)
            hip.hipGraphDestroy(graph)
