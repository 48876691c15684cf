"""Tracing rules (lumen/graph/tracer.py): dtypes without implicit promotion, weak Python scalars, type
inference errors with the reference's messages, and errors for closures over data and data-dependent control
flow."""

import pytest

import lumen_amd as L
import lumen_amd.functional as F
from lumen_amd.graph.ir import Graph, InferError


def _g(fn, *metas):
    return L.make_graph(fn)(*[L.empty(list(s), d, "meta") for s, d in metas])


def test_weak_scalars_take_the_tensor_dtype():
    g = _g(lambda x: x * 2.0 + 1, ((3,), "bfloat16"))
    assert all(g.types[n.output].dtype in ("bfloat16", "bool") for n in g.nodes if n.prim != "iota")


def test_mixed_dtypes_raise():
    with pytest.raises(TypeError, match="convert them to one"):
        _g(lambda x, y: x + y, ((3,), "float32"), ((3,), "bfloat16"))


def test_matmul_needs_explicit_dtypes():
    with pytest.raises(TypeError, match="@ has no dtypes"):
        _g(lambda x: x @ x, ((3, 3), "float32"))


def test_dot_general_output_dtype_is_accumulator_then_cast():
    g = _g(lambda x, w: F.matmul(x, w, "float32", "bfloat16"), ((2, 4), "bfloat16"), ((4, 3), "bfloat16"))
    prims_ = [n.prim for n in g.nodes]
    assert prims_ == ["dot_general", "cast"]
    assert g.types[g.nodes[0].output].dtype == "float32"


def test_infer_errors_name_the_primitive():
    g = Graph()
    a = g.input("float32", (2, 3))
    b = g.input("float32", (3, 2))
    with pytest.raises(InferError, match="add: operands must have the same type"):
        g.apply("add", [a, b])
    c = g.input("int32", (2,))
    with pytest.raises(InferError, match="ambiguous"):
        g.apply("cast", [c], {"new_dtype": "bfloat16"})
    with pytest.raises(InferError, match="accumulates in the operand's dtype"):
        g.apply("reduce_sum", [a], {"axes": (0,), "accum_dtype": "float64"})


def test_control_flow_on_traced_values_raises():
    with pytest.raises(TypeError, match="no value"):
        _g(lambda x: x * 2.0 if x else x, ((1,), "float32"))


def test_closing_over_a_tensor_raises():
    t = L.ones([3])
    with pytest.raises(TypeError, match="cannot close over a tensor"):
        _g(lambda x: x + t, ((3,), "float32"))


def test_prune_drops_dead_nodes_and_keeps_inputs():
    g = _g(lambda x, y: (F.exp(x), F.log(y))[0], ((3,), "float32"), ((3,), "float32"))
    assert [n.prim for n in g.nodes] == ["exp"]
    assert len(g.inputs) == 2


def test_module_weights_and_written_outputs():
    from lumen_amd.graph.trace import trace

    class M(L.nn.Module):
        w: L.Tensor
        lr: float

        def step(self, x):
            loss = F.sum(self.w * x)
            loss.backward()
            self.w.copy_(self.w - self.lr * self.w.grad)
            return loss

    m = M(L.empty([3], "float32", "meta"), 0.5)
    t = trace(lambda m, x: m.step(x), (m, L.empty([3], "float32", "meta")))
    kinds = [k for k, _ in t.layout]
    assert kinds == ["arg", "scalar", "weight"]
    assert t.written == [0] and len(t.graph.outputs) == 2


def test_to_with_an_unknown_device_string_names_the_device():
    """``t.to("cuda")`` on a traced tensor raises the unknown-device error (this backend's GPU is ``hip``),
    not a dtype error; known devices and dtype names still work."""
    import pytest

    with pytest.raises(ValueError, match="unknown device 'cuda'"):
        L.make_graph(lambda x: x.to("cuda"))(L.empty([2], "float32", "meta"))
    g = L.make_graph(lambda x: x.to("hip:0").to("bfloat16"))(L.empty([2], "float32", "meta"))
    assert [n.prim for n in g.nodes] == ["cast"]
