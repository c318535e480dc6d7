"""include/qmsg.h from C: every C block of INTEGRATION.md compiled with gcc -std=gnu11 -Wall
-Werror and linked against libqmsg.so (tests/c_consumer/main.c drives them).

The blocks are taken as a maintainer would paste them into src/model.c: file-level blocks as
they stand, the call-site patch as its "+" lines inside a function with qms_forward's locals
(src/model.c:1284), statement fragments inside functions whose parameters name what they use.
Where the reference's sources are present, its model.h supplies QmsModel for the in-RAM attach.
Without a GPU the program reports QMSG_E_DEVICE; on the GPU it attaches a written model file
and the call site's output equals the oracle's layer bit for bit."""
import os
import re
import shutil
import subprocess

import numpy as np
import pytest

import gguf_file as gf
import oracle as orc

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
REF_SRC = "/root/reference/src"
FRAGMENT_ARGS = ("qmsg_gguf *g, int l, int T, const QmsCfg *c, float *d_h, const float *d_xn, "
                 "float *d_q, float *d_k, float *d_v")


def c_blocks(text):
    return re.findall(r"```c\n(.*?)```", text, re.S)


def snippets(with_qms):
    """The translation unit INTEGRATION.md's C blocks make, plus snippets_mark_used()."""
    out, used = [], []
    for i, b in enumerate(c_blocks(open(os.path.join(ROOT, "INTEGRATION.md")).read())):
        lines = b.rstrip("\n").split("\n")
        needs_qms = "Qms" in b or "c->" in b
        if needs_qms and not with_qms:
            continue
        if all(l[:1] in "+-" for l in lines if l.strip()):                 # the call-site patch
            body = "\n".join(l[1:] for l in lines if l.startswith("+"))
            out.append("static int qmsg_call_site(int l, float *xn, float *h, int T, float *tmp)\n{\n"
                       + body + "\n    return 0;\n}\n")
            used.append("qmsg_call_site")
        elif re.search(r"^(static )?\w[\w\s\*]*\b(\w+)\([^;]*\)\s*\{", b, re.M) or b.lstrip().startswith("#"):
            out.append(b)                                                   # file-level
            used += re.findall(r"^static int (\w+)\(", b, re.M)
        else:                                                               # statement fragment
            args = FRAGMENT_ARGS if with_qms else FRAGMENT_ARGS.replace("const QmsCfg *c, ", "")
            out.append(f"void integration_fragment_{i}({args})\n{{\n{b}}}\n")
    mark = "static void snippets_mark_used(void)\n{\n" + "".join(f"    (void)&{u};\n" for u in used) + "}\n"
    return "\n".join(out) + "\n" + mark, used


def build(tmp_path, with_qms):
    gcc = shutil.which("gcc")
    lib = os.path.join(ROOT, "large_model_amd", "libqmsg.so")
    if gcc is None or not os.path.exists(lib):
        pytest.skip("gcc or the built libqmsg.so is missing")
    src, used = snippets(with_qms)
    assert {"qmsg_attach_file", "qmsg_call_site"} <= set(used)
    if with_qms:
        assert "qmsg_attach" in used
    (tmp_path / "snippets.inc").write_text(src)
    exe = str(tmp_path / "consumer")
    cmd = [gcc, "-std=gnu11", "-Wall", "-Werror", "-O1", "-I", os.path.join(ROOT, "include"), "-I", str(tmp_path)]
    if with_qms:
        cmd += ["-DQMSG_WITH_QMS", "-D_GNU_SOURCE", "-isystem", REF_SRC]
    cmd += [os.path.join(ROOT, "tests", "c_consumer", "main.c"), "-o", exe, "-L", os.path.dirname(lib), "-lqmsg",
            "-Wl,-rpath," + os.path.dirname(lib)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr + "\n" + src
    return exe


def test_snippets_compile_and_report_no_device(tmp_path):
    from conftest_gpu import gpu_available
    with_qms = os.path.exists(os.path.join(REF_SRC, "model.h"))
    exe = build(tmp_path, with_qms)
    r = subprocess.run([exe, "probe"], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    if gpu_available():
        assert r.stdout.startswith("status 0 "), r.stdout
    else:
        assert r.stdout.startswith("status -4 "), r.stdout             # QMSG_E_DEVICE


def test_call_site_error_path_without_device(tmp_path):
    """No GPU: the attach snippet prints the library's reason and the program stops there."""
    from conftest_gpu import gpu_available
    if gpu_available():
        pytest.skip("a GPU is present")
    exe = build(tmp_path, False)
    lays = [orc.Layer(256, 16, 4, 256, 41, layer=0)]
    path, _ = gf.moe_model(str(tmp_path / "m.gguf"), lays)
    x = orc.make_input(256, 2, 3)
    x.tofile(str(tmp_path / "x.f32"))
    r = subprocess.run([exe, "run", path, "0", "2", str(tmp_path / "x.f32"), str(tmp_path / "o.f32")],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 3 and r.stderr.startswith("qmsg: "), (r.returncode, r.stderr)


@pytest.mark.gpu
@pytest.mark.parametrize("T", [1, 5, 40])
def test_call_site_equals_oracle(tmp_path, T):
    print(f"[case] C consumer T={T}", flush=True)
    exe = build(tmp_path, os.path.exists(os.path.join(REF_SRC, "model.h")))
    lays = [orc.Layer(256, 16, 4, 256, 50 + l, layer=l, down_type=dt)
            for l, dt in enumerate((orc.T_Q4_0, orc.T_Q6_K))]
    path, _ = gf.moe_model(str(tmp_path / "m.gguf"), lays, n_shards=2)
    x = orc.make_input(256, T, 7 + T)
    x.tofile(str(tmp_path / "x.f32"))
    for l, lay in enumerate(lays):
        out_path = str(tmp_path / f"o{l}.f32")
        r = subprocess.run([exe, "run", path, str(l), str(T), str(tmp_path / "x.f32"), out_path],
                           capture_output=True, text=True, timeout=120)
        assert r.returncode == 0, r.stderr
        got = np.fromfile(out_path, dtype=np.float32).reshape(T, 256)
        assert np.array_equal(got.view(np.uint32), lay.moe(x).view(np.uint32)), l
