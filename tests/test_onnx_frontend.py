"""compiler/onnx_reader.py on ONNX wire-format files written by
tests/onnx_writer.py (CPU only): the exported ResNet-18 / LeNet-5 / encoder
graphs come back with the same nodes, constants and O1 call sequence,
Conv + BatchNormalization is folded like the reference's onnxsim step, and
Compiler(...).compile() takes an .onnx path."""

from __future__ import annotations

import numpy as np
import pytest

import onnx_writer


def _calls(graph, opt=1):
    """op and non-tensor arguments of every call; float arguments as fp32
    (ONNX stores float attributes as fp32, as the C code does)."""
    from nnc_py_amd.compiler import build_program
    norm = lambda a: ("f", float(np.float32(a[1]))) if a[0] == "f" else a
    return [(c.op, [norm(a) for a in c.args if a[0] != "t"]) for c in build_program(graph, opt_level=opt).calls]


@pytest.mark.parametrize("model", ["resnet18", "lenet5", "encoder"])
def test_roundtrip_through_onnx(model, tmp_path, pkg):
    from nnc_py_amd.compiler import zoo
    from nnc_py_amd.compiler.onnx_reader import load_onnx
    make = {"resnet18": lambda: zoo.resnet18(batch=1, seed=0), "lenet5": lambda: zoo.lenet5(batch=1, seed=0),
            "encoder": lambda: zoo.transformer_encoder(batch=1, seq=8, seed=0)}[model]
    path = tmp_path / f"{model}.onnx"
    path.write_bytes(onnx_writer.from_graph(make()))
    g = load_onnx(path)
    ref = make()
    assert [n.op_type for n in g.nodes] == [n.op_type for n in ref.nodes]
    assert [n.name for n in g.nodes] == [n.name for n in ref.nodes]
    for k, t in ref.constants.items():
        assert np.array_equal(g.constants[k].data, t.data), k
    assert _calls(g) == _calls(make())


def test_conv_batchnorm_folding(tmp_path, pkg, oracle_lib):
    from nnc_py_amd.compiler import Executor, build_program
    from nnc_py_amd.compiler.onnx_reader import load_onnx
    rng = np.random.default_rng(0)
    w = rng.standard_normal((8, 3, 3, 3)).astype(np.float32)
    bias = rng.standard_normal(8).astype(np.float32)
    gamma, beta = rng.uniform(0.5, 1.5, 8).astype(np.float32), rng.standard_normal(8).astype(np.float32)
    mean, var = rng.standard_normal(8).astype(np.float32), rng.uniform(0.5, 2, 8).astype(np.float32)
    nodes = [onnx_writer.node("Conv", ["x", "w", "b"], ["c"], "conv", kernel_shape=[3, 3], pads=[1, 1, 1, 1],
                              strides=[1, 1]),
             onnx_writer.node("BatchNormalization", ["c", "g", "be", "m", "v"], ["bn"], "bn", epsilon=1e-5),
             onnx_writer.node("Relu", ["bn"], ["y"], "relu")]
    data = onnx_writer.model(nodes, {"w": w, "b": bias, "g": gamma, "be": beta, "m": mean, "v": var},
                             [("x", (1, 3, 8, 8))], [("y", (1, 8, 8, 8))])
    path = tmp_path / "cbr.onnx"
    path.write_bytes(data)
    g = load_onnx(path)
    assert [n.op_type for n in g.nodes] == ["Conv", "Relu"]
    x = rng.standard_normal((1, 3, 8, 8)).astype(np.float32)
    ex = Executor(build_program(g, opt_level=1), device=False, lib=oracle_lib)
    ex.set_input("x", x)
    ex.run()
    # float64: convolution, then batch norm, then relu
    xp = np.pad(x.astype(np.float64), ((0, 0), (0, 0), (1, 1), (1, 1)))
    conv = np.zeros((8, 8, 8))
    for co in range(8):
        for r in range(3):
            for c in range(3):
                conv[co] += np.einsum("chw,c->hw", xp[0, :, r:r + 8, c:c + 8], w[co, :, r, c].astype(np.float64))
        conv[co] += bias[co]
    bn = (conv - mean[:, None, None]) / np.sqrt(var[:, None, None] + 1e-5) * gamma[:, None, None] + beta[:, None, None]
    want = np.maximum(bn, 0)[None]
    np.testing.assert_allclose(ex.get("y"), want, rtol=1e-4, atol=1e-4)


def test_compiler_accepts_an_onnx_path(tmp_path, pkg):
    from nnc_py_amd.compiler import zoo
    from nnc_py_amd.compiler.compiler import Compiler
    path = tmp_path / "lenet.onnx"
    path.write_bytes(onnx_writer.from_graph(zoo.lenet5(batch=1, seed=0)))
    prog = Compiler(target="mi355x", opt_level=3).compile(str(path), str(tmp_path / "out"))
    assert (tmp_path / "out" / "model.c").exists() and prog.calls


def test_symbolic_input_needs_a_shape(tmp_path, pkg):
    from nnc_py_amd.compiler.onnx_reader import load_onnx
    import onnx_writer as w
    data = w.model([w.node("Relu", ["x"], ["y"], "r")], {}, [("x", (0, 4))], [("y", (0, 4))])
    path = tmp_path / "sym.onnx"
    path.write_bytes(data)
    with pytest.raises(ValueError):
        load_onnx(path)
    g = load_onnx(path, input_shapes={"x": (2, 4)})
    assert g.tensors["y"].shape == (2, 4)
