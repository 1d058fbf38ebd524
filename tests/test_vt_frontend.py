"""The .vt front end of compile-train (include/volta_vt.h) and the volta-hip
command line, on the CPU: what spec each source resolves to on either code
path, the guards, the reference's own example scripts, the command line's
argument rules and the generated per-model library's exports."""
import ctypes as C
import os
import subprocess

import pytest

from volta_amd import HIP_LIB, load_hip
from volta_amd.abi import ACTIVATIONS, OPTIMIZERS, CSpec

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CLI = os.path.join(ROOT, "volta_amd", "volta-hip")
pytestmark = pytest.mark.skipif(not (os.path.exists(HIP_LIB) and os.path.exists(CLI)),
                                reason="library / CLI not built")

HEADLINE = """# the headline topology with Adam
model net
    layers 512 1024 1024 512 256 1
    activation relu

dataset data
    type synthetic
    batch 64

train net on data
    epochs 50
    optimizer adam
    lr 0.001
    device cpu
"""


def resolve(source):
    lib = load_hip()
    spec = CSpec()
    buf = C.create_string_buffer(4096)
    rc = lib.lib.volta_vt_compile_train_spec(source.encode(), C.byref(spec), buf, len(buf))
    if rc != 0:
        raise ValueError(lib.last_error())
    return spec, buf.value.decode()


def names(spec):
    act = {v: k for k, v in ACTIVATIONS.items()}[spec.activation]
    opt = {v: k for k, v in OPTIMIZERS.items()}[spec.optimizer]
    return list(spec.sizes[:spec.n_sizes]), act, opt


def test_headline_source():
    spec, summary = resolve(HEADLINE)
    assert names(spec) == ([512, 1024, 1024, 512, 256, 1], "relu", "adam")
    assert spec.loss == 0 and abs(spec.beta1 - 0.9) < 1e-7 and abs(spec.eps - 1e-8) < 1e-12
    assert "lr=0.001 epochs=50 batch=64" in summary
    assert "note: the reference trains the model in its interpreter for 50 epoch(s)" in summary


@pytest.mark.parametrize("src,want", [
    # no train statement: the model's own optimizer, else SGD (executor.rs:1834-1837)
    ("model m\n    layers 4 8 2\n", ([4, 8, 2], "relu", "sgd")),
    ("model m\n    layers 4 8 2\n    activation tanh\n    optimizer adagrad 0.01\n", ([4, 8, 2], "tanh", "adagrad")),
    # train without optimizer: autopilot rule, adam up to 6 layers, adamw above
    ("model m\n    layers 4 8 2\ndataset d\ntrain m on d\n", ([4, 8, 2], "relu", "adam")),
    ("model m\n    layers 4 8 8 8 8 8 8 2\ndataset d\ntrain m on d\n", ([4, 8, 8, 8, 8, 8, 8, 2], "relu", "adamw")),
    # train optimizer beats the model's; the last train statement decides
    ("model m\n    layers 4 8 2\n    optimizer sgd\ndataset d\ntrain m on d\n    optimizer adamw\n"
     "train m on d\n    optimizer Adagrad\n", ([4, 8, 2], "relu", "adagrad")),
    # aliases, variables, comments, strings and negative numbers
    ("width 16  # a variable\nmodel m  # comment\n    layers 4 width 2\n    activation leakyrelu\n"
     "    seed -3\ndataset d\n    source \"x.csv\"\ntrain m on d\n    optimizer sgd\n",
     ([4, 16, 2], "leaky_relu", "sgd")),
    ("model m\n    layers 4 8 2\n    activation softmax\n", ([4, 8, 2], "softmax", "sgd")),
    # the first model is the one compiled
    ("model a\n    layers 3 5 1\n    activation gelu\nmodel b\n    layers 9 9 9\n", ([3, 5, 1], "gelu", "sgd")),
])
def test_resolution(src, want):
    spec, _ = resolve(src)
    assert names(spec) == want


@pytest.mark.parametrize("src,msg", [
    ("model m\n    layers 4 8 2\ndataset d\ntrain m on d\n    optimizer rmsprop\n",
     "supports only SGD, Adam, AdamW, and Adagrad"),
    ("model m\n    layers 4 8 2\n    use block\n", "is MLP-only"),
    ("model m\n    layers 4 8 2\n    dropout 1.0\n", "model.dropout must be in [0, 1)"),
    ("model m\n    layers 4 8 2\ndataset d\ntrain m on d\n    clip_grad 0\n", "clip_grad must be positive"),
    ("model m\n    layers 4 8 2\n    activation swish\n", "invalid value 'swish'"),
    ("model m\n    layers 4\n", "at least 2 values"),
    ("model m\n    layers 4 0 2\n", "must be > 0"),
    ("model m\n    activation relu\n", "missing required property 'layers'"),
    ("model m\n    layers 4 8 2\n    layers 4 8 2\n", "duplicate 'layers'"),
    ("model m\n\tlayers 4 8 2\n", "tabs are not allowed"),
    ("model m\n  layers 4 8 2\n", "inconsistent indentation"),
    ("model m\n    layers 4 8 2\ntrain m on nowhere\n", "Undefined dataset: 'nowhere'"),
    ("dataset d\n", "No models found"),
    ("// a comment the language does not have\nmodel m\n    layers 4 8 2\n",
     "Unexpected token at start of statement"),
    ("model m\n    layers 4 8 2\nelse\n    print 1\n", "Unexpected keyword in this position"),
])
def test_guards(src, msg):
    with pytest.raises(ValueError) as e:
        resolve(src)
    assert msg in str(e.value), str(e.value)


@pytest.mark.parametrize("src,want", [
    # model.dropout / model.layernorm (executor.rs:1930-1971)
    ("model m\n    layers 4 8 2\n    dropout 0.25\n    layernorm yes\n", (0.0, 0.25, 1)),
    ("model m\n    layers 4 8 2\n    layernorm no\n    dropout 0\n", (0.0, 0.0, 0)),
    ("model m\n    layers 4 8 2\n    layernorm on\n", (0.0, 0.0, 1)),
    # the last run of the model that sets clip_grad keeps it (executor.rs:1299)
    ("model m\n    layers 4 8 2\ndataset d\ntrain m on d\n    clip_grad 2.5\ntrain m on d\n    epochs 1\n",
     (2.5, 0.0, 0)),
    ("model m\n    layers 4 8 2\nmodel k\n    layers 2 2\ndataset d\ntrain m on d\n    clip_grad 2.5\n"
     "train m on d\n    clip_grad 0.5\ntrain k on d\n    clip_grad 9\n", (0.5, 0.0, 0)),
])
def test_codegen_extras(src, want):
    spec, summary = resolve(src)
    assert (round(spec.clip_grad, 6), round(spec.dropout_p, 6), spec.layernorm) == want
    if want[2]:
        assert "layernorm=yes" in summary


def test_statements_outside_compile_train_are_noted_not_run():
    """Every other statement of the language is parsed structurally and
    noted (the reference's interpreter runs it before compiling the first
    model, main.rs:224-246); the model resolves as without it."""
    src = ("lr 0.01\nfn f(x)\n    print x\n    return x + 1\nif lr > 0.005\n    print \"high\"\n"
           "elif lr > 0.001\n    print \"mid\"\nelse\n    print \"low\"\nfor i in 0..3\n    print i\n"
           "loop 2\n    print 1\nprint f(5)\nmodel m\n    layers 4 8 2\n    activation tanh\n"
           "dataset d\n    batch 4\ntrain m on d\n    optimizer sgd\n    lr lr\n"
           "save m \"m.bin\"\ninfer m\n    input 1 2 3 4\n")
    spec, summary = resolve(src)
    assert names(spec) == ([4, 8, 2], "tanh", "sgd")
    for kw in ("fn", "if", "elif", "else", "for", "loop", "save", "infer"):
        assert f"'{kw}' statement not run" in summary, kw
    assert "lr=0.01" in summary


def test_c_path_resolution():
    """Without --rust the reference's C path: SGD only (its own message),
    ReLU hidden layers, MSE and no codegen extras whatever the model says
    (mlp_train_codegen.rs:291-384), each dropped property noted."""
    lib = load_hip()

    def resolve_c(src):
        spec = CSpec()
        buf = C.create_string_buffer(4096)
        if lib.lib.volta_vt_compile_train_spec_path(src.encode(), 0, C.byref(spec), buf, len(buf)) != 0:
            raise ValueError(lib.last_error())
        return spec, buf.value.decode()

    spec, summary = resolve_c("model m\n    layers 4 8 2\n    activation gelu\n    dropout 0.5\n"
                              "    layernorm yes\ndataset d\ntrain m on d\n    optimizer sgd\n    clip_grad 1\n")
    assert names(spec) == ([4, 8, 2], "relu", "sgd") and spec.loss == 0
    assert (spec.clip_grad, spec.dropout_p, spec.layernorm) == (0.0, 0.0, 0)
    assert "path=c" in summary and "activation 'gelu' applies with --rust only" in summary
    assert "no dropout, LayerNorm or gradient clipping" in summary
    with pytest.raises(ValueError) as e:
        resolve_c("model m\n    layers 4 8 2\ndataset d\ntrain m on d\n    optimizer adam\n")
    assert "the default C compile-train path supports only SGD today" in str(e.value)


REF_EXAMPLES = "/root/reference/examples"
EXAMPLES_WANT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "vt_examples.json")


@pytest.mark.skipif(not os.path.isdir(REF_EXAMPLES), reason="reference examples not mounted")
@pytest.mark.parametrize("path", ["c", "rust"])
def test_reference_examples(path):
    """The reference's own example scripts (examples/*.vt, read where they
    lie) against a table written by hand from reading them: layers,
    activation, optimizer, lr, epochs and batch per path, or the error the
    reference's parser or guards give (five examples open with `//` lines,
    which its lexer reads as two Slash tokens: "Unexpected token at start of
    statement", parser.rs:83-86)."""
    import glob
    import json

    want = json.load(open(EXAMPLES_WANT))
    files = sorted(glob.glob(os.path.join(REF_EXAMPLES, "*.vt")))
    assert sorted(os.path.basename(f) for f in files) == sorted(want), "example set changed"
    for f in files:
        w = want[os.path.basename(f)]
        r = subprocess.run([CLI, "check", f] + (["--rust"] if path == "rust" else []), capture_output=True,
                           text=True)
        exp = w.get(path, w.get("both"))
        if "error" in exp:
            assert r.returncode == 1 and exp["error"] in r.stderr, (f, r.stderr)
            continue
        assert r.returncode == 0, (f, r.stderr)
        line = r.stdout.splitlines()[0]
        fields = dict(kv.split("=", 1) for kv in line.split())
        for k, v in exp.items():
            assert fields.get(k) == v, (f, k, fields.get(k), v)


def test_cli_flags_as_the_reference_checks_them(tmp_path):
    """compile-train's arguments (main.rs:587-650): -o once, --rust once,
    --cpu-target portable|native (separate or =), no other flag, one file."""
    vt = tmp_path / "net.vt"
    vt.write_text(HEADLINE)
    cases = [
        (["--rust", "--rust"], "accepts '--rust' at most once"),
        (["--cpu-target", "fast"], "accepts only 'portable' or 'native', got 'fast'"),
        (["--cpu-target"], "requires 'portable' or 'native'"),
        (["-o"], "requires an output path"),
        (["-o", "a.so", "-o", "b.so"], "accepts '-o' at most once"),
        (["--frobnicate"], "does not accept flag '--frobnicate'"),
        ([str(vt)], "expects exactly one .vt file"),
    ]
    for extra, msg in cases:
        r = subprocess.run([CLI, "compile-train", str(vt)] + extra, capture_output=True, text=True)
        assert r.returncode == 2 and msg in r.stderr, (extra, r.stderr)
    r = subprocess.run([CLI, "compile-train"], capture_output=True, text=True)
    assert r.returncode == 2
    for flags, name in ((["--rust", "--cpu-target=native"], "net.train_rust.so"),
                        (["--cpu-target", "portable", "--rust"], "net.train_rust.so")):
        r = subprocess.run([CLI, "compile-train", str(vt)] + flags, capture_output=True, text=True)
        assert r.returncode == 0, r.stderr
        assert r.stdout.startswith(f"Training DLL compiled: {tmp_path / name} (cpu-target=")
        assert (tmp_path / name).exists()
    # the C path refuses Adam with the reference's message
    r = subprocess.run([CLI, "compile-train", str(vt)], capture_output=True, text=True)
    assert r.returncode == 1 and "supports only SGD today" in r.stderr


def test_cli_weights_export_load_pretrained(tmp_path):
    """--weights embeds trained parameters and exports
    volta_train_load_pretrained (the C path's loader,
    mlp_train_codegen.rs:386-413); a file of the wrong size is refused."""
    import numpy as np

    vt = tmp_path / "m.vt"
    vt.write_text("model m\n    layers 4 3 2\n")
    w = tmp_path / "m.f32"
    np.arange(4 * 3 + 3 + 3 * 2 + 2, dtype=np.float32).tofile(w)
    r = subprocess.run([CLI, "compile-train", str(vt), "--weights", str(w)], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    lib = C.CDLL(str(tmp_path / "m.train.so"))
    assert hasattr(lib, "volta_train_load_pretrained")
    r = subprocess.run([CLI, "compile-train", str(vt), "-o", str(tmp_path / "plain.so")], capture_output=True,
                       text=True)
    assert r.returncode == 0, r.stderr
    assert not hasattr(C.CDLL(str(tmp_path / "plain.so")), "volta_train_load_pretrained")
    np.zeros(5, np.float32).tofile(w)
    r = subprocess.run([CLI, "compile-train", str(vt), "--weights", str(w)], capture_output=True, text=True)
    assert r.returncode == 1 and "holds 20 bytes" in r.stderr


def test_cli_check_and_compile_train(tmp_path):
    vt = tmp_path / "net.vt"
    vt.write_text(HEADLINE)
    r = subprocess.run([CLI, "check", str(vt), "--rust"], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    assert r.stdout.startswith("model=net path=rust layers=512-1024-1024-512-256-1 activation=relu optimizer=adam")
    bad = tmp_path / "bad.vt"
    bad.write_text("model m\n    layers 4 8 2\ndataset d\ntrain m on d\n    optimizer rmsprop\n")
    r = subprocess.run([CLI, "compile-train", str(bad), "--rust"], capture_output=True, text=True)
    assert r.returncode == 1 and "rmsprop" in r.stderr
    r = subprocess.run([CLI, "compile-train", str(vt), "--rust"], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    out = tmp_path / "net.train_rust.so"
    assert out.exists() and not (tmp_path / "net.train_rust.so.c").exists()
    lib = C.CDLL(str(out))
    for sym in ("volta_train_init", "volta_train_step", "volta_train_loss", "volta_train_get_params",
                "volta_train_set_params", "volta_train_free", "volta_train_step_labels"):
        assert hasattr(lib, sym), sym
    lib.volta_train_init.restype = C.c_void_p
    lib.volta_train_last_error.restype = C.c_char_p
    h = lib.volta_train_init(8)  # no GPU here: NULL with the library's reason
    if h:
        lib.volta_train_free.argtypes = [C.c_void_p]
        lib.volta_train_free(h)
    else:
        assert b"HIP" in lib.volta_train_last_error()
    r = subprocess.run([CLI, "compile-train", str(vt), "--rust", "-o", str(tmp_path / "x.so"), "--keep-source"],
                       capture_output=True, text=True)
    assert r.returncode == 0 and (tmp_path / "x.so.c").exists()
    assert subprocess.run([CLI, "frobnicate", str(vt)], capture_output=True).returncode == 2


INFER_VT = "model m\n    layers 4 3 2\n    activation {act}\n\ndataset d\n    batch 2\n\ntrain m on d\n    epochs 1\n" \
           "    optimizer rmsprop\n"


def _rodata(path):
    """The bytes of a shared library's .rodata section."""
    import tempfile

    with tempfile.NamedTemporaryFile(suffix=".bin") as f:
        subprocess.run(["objcopy", "-O", "binary", "--only-section=.rodata", str(path), f.name], check=True)
        return open(f.name, "rb").read()


def test_compile_flags_as_the_reference_checks_them(tmp_path):
    """compile's arguments (main.rs:541-586): -o once and not a flag,
    --cpu-target portable|native, no other flag, exactly one file."""
    vt = tmp_path / "m.vt"
    vt.write_text(INFER_VT.format(act="relu"))
    cases = [
        (["--cpu-target", "fast"], "'compile --cpu-target' accepts only 'portable' or 'native', got 'fast'"),
        (["-o"], "'compile -o' requires an output path"),
        (["-o", "--rust"], "'compile -o' requires an output path"),
        (["-o", "a.so", "-o", "b.so"], "'compile' accepts '-o' at most once"),
        (["--rust"], "'compile' does not accept flag '--rust'"),
        ([str(vt)], "'compile' expects exactly one .vt file"),
    ]
    for extra, msg in cases:
        r = subprocess.run([CLI, "compile", str(vt)] + extra, capture_output=True, text=True)
        assert r.returncode == 2 and msg in r.stderr, (extra, r.stderr)
    r = subprocess.run([CLI, "compile"], capture_output=True, text=True)
    assert r.returncode == 2 and "'compile' expects a .vt file path" in r.stderr


@pytest.mark.parametrize("act,ok", [("relu", True), ("gelu", True), ("tanh", True), ("sigmoid", False),
                                    ("softmax", False)])
def test_compile_resolution(tmp_path, act, ok):
    """The inference graph of lower_model_to_graph (lowering.rs:87-140): ReLU
    hidden layers for 'relu', linear for the activations it drops (noted);
    'sigmoid' and 'softmax' fail as the reference's inference codegen fails
    on Sigmoid / Softmax nodes (codegen/inner.rs:395-399).  No compile-train
    optimizer guard applies (the script trains with RMSProp here)."""
    import numpy as np

    vt = tmp_path / "m.vt"
    vt.write_text(INFER_VT.format(act=act))
    w = tmp_path / "m.f32"
    np.arange(4 * 3 + 3 + 3 * 2 + 2, dtype=np.float32).tofile(w)
    r = subprocess.run([CLI, "compile", str(vt), "--weights", str(w)], capture_output=True, text=True)
    if not ok:
        assert r.returncode == 1 and "Unsupported op in codegen" in r.stderr, r.stderr
        return
    assert r.returncode == 0, r.stderr
    assert r.stdout.startswith(f"Compiled: {tmp_path / 'm.so'} (cpu-target=portable)")
    assert ("no activation for '%s'" % act in r.stdout) == (act != "relu")


def test_compile_requires_weights_and_checks_their_size(tmp_path):
    import numpy as np

    vt = tmp_path / "m.vt"
    vt.write_text(INFER_VT.format(act="relu"))
    r = subprocess.run([CLI, "compile", str(vt)], capture_output=True, text=True)
    assert r.returncode == 1 and "Model 'm' has no weights" in r.stderr
    w = tmp_path / "m.f32"
    np.zeros(5, np.float32).tofile(w)
    r = subprocess.run([CLI, "compile", str(vt), "--weights", str(w)], capture_output=True, text=True)
    assert r.returncode == 1 and "holds 20 bytes" in r.stderr and "needs 92" in r.stderr


def test_compile_library_embeds_weights_and_exports_volta_infer(tmp_path):
    """The generated library carries the weights file's bytes in its
    read-only data (the reference embeds its trained weights as constant
    globals, codegen/inner.rs:251-260) -- also from a path holding a quote,
    a backslash and a newline -- and exports volta_infer.  Without a GPU the
    first call writes nothing and names the reason."""
    import numpy as np

    vt = tmp_path / "m.vt"
    vt.write_text(INFER_VT.format(act="relu"))
    blob = np.random.default_rng(3).standard_normal(4 * 3 + 3 + 3 * 2 + 2).astype(np.float32)
    w = tmp_path / 'w"e\\ir\nd.f32'
    blob.tofile(w)
    out = tmp_path / "inf.so"
    r = subprocess.run([CLI, "compile", str(vt), "--weights", str(w), "-o", str(out)], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    assert blob.tobytes() in _rodata(out)
    lib = C.CDLL(str(out))
    assert hasattr(lib, "volta_infer")
    F = C.POINTER(C.c_float)
    lib.volta_infer.argtypes = [F, C.c_int64, F, C.c_int64]
    lib.volta_infer_last_error.restype = C.c_char_p
    X = np.ones(4, np.float32)
    y = np.full(2, 5.0, np.float32)
    lib.volta_infer(X.ctypes.data_as(F), 4, y.ctypes.data_as(F), 2)
    if lib.volta_infer_last_error():  # no GPU here
        assert (y == 5.0).all() and b"HIP" in lib.volta_infer_last_error()


def test_compile_train_weights_rounded_as_the_reference_literals(tmp_path):
    """compile-train --weights embeds each value as the reference's C-path
    loader holds it: printed f"{v:.8}f" (mlp_train_codegen.rs:393-405) and
    read back as the nearest float32 -- values below 5e-9 become 0, and
    others move by up to 5e-9."""
    import numpy as np

    vt = tmp_path / "m.vt"
    vt.write_text("model m\n    layers 4 3 2\n")
    blob = np.random.default_rng(4).standard_normal(4 * 3 + 3 + 3 * 2 + 2).astype(np.float32)
    blob[:4] = [1e-9, -3e-9, 0.123456789, 2.0 ** -9 * 63]
    w = tmp_path / "m.f32"
    blob.tofile(w)
    r = subprocess.run([CLI, "compile-train", str(vt), "--weights", str(w), "-o", str(tmp_path / "t.so")],
                       capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    want = np.array([np.float32(f"{float(v):.8f}") for v in blob], np.float32)
    assert want[0] == 0 and want[1] == 0 and want[2] == np.float32(0.12345679)
    assert want.tobytes() in _rodata(tmp_path / "t.so")
    assert not (tmp_path / "t.so.weights").exists()
