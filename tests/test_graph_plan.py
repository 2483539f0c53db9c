"""Graph planning on the CPU (no GPU needed): the library compiles a node list without a session and
reports its passes, which follow the reference's rules case for case.

- fuseMatMulBias (graph/fuse_matmul_bias.go:12-63): MatMul(x, W const f32 2-D) → Add(const f32 [N]) folds into
  a 3-input MatMul when the product's sole consumer is that Add and the product is not a graph output.
- planHalf (graph/gpuhalf_darwin_arm64.go:29-112): a Gemm/MatMul against a constant f32 2-D weight whose sole
  consumer (slot 0) is Relu, Sigmoid, SiLU or Gelu applies it in its store; under GPUBF16 every such product
  runs bf16 and stores bf16 exactly when every reader of its value is such a product reading slot 0.
"""
import pytest

from ingot_amd import Graph, IngotError
from ingot_amd import _lib as L

F = L.GRAPH_FUSE_BIAS | L.GRAPH_FUSE_ACT | L.GRAPH_HALF


def plan(text, flags):
    g = Graph(None, text)
    g.compile(flags)
    out = g.stats(), {ln.split(" ")[0] + ":" + ln.split("out=")[1].split(" ")[0]: ln for ln in g.plan()}
    g.free()
    return out


def field(line, key):
    return line.split(key + "=")[1].split(" ")[0]


MLP = """
input x f32 128,768
const W1 f32 768,3072
const b1 f32 3072
const W2 f32 3072,768
const b2 f32 768
node MatMul x,W1 -> h1
node Add h1,b1 -> h2
node ingot.Gelu h2 -> h3
node MatMul h3,W2 -> h4
node Add b2,h4 -> h5
node Relu h5 -> y
output y
"""


def test_fuse_matmul_bias_both_add_orders():
    st, p = plan(MLP, L.GRAPH_FUSE_BIAS)
    assert st["fuse-matmul-bias"] == 2 and st["steps"] == 4
    assert field(p["MatMul:h2"], "in") == "x,W1,b1"
    assert field(p["MatMul:h5"], "in") == "h3,W2,b2"          # Add(bias, product) order too
    assert "Add:h2" not in p and "Add:h5" not in p


@pytest.mark.parametrize("case,text", [
    ("weight not constant", MLP.replace("const W1 f32 768,3072", "input W1 f32 768,3072")),
    ("weight not f32", MLP.replace("const W1 f32 768,3072", "const W1 bf16 768,3072")),
    ("weight not 2-D", MLP.replace("const W1 f32 768,3072", "const W1 f32 1,768,3072")),
    ("bias not constant", MLP.replace("const b1 f32 3072", "input b1 f32 3072")),
    ("bias length", MLP.replace("const b1 f32 3072", "const b1 f32 768")),
    ("bias not trailing", MLP.replace("const b1 f32 3072", "const b1 f32 3072,1")),
    ("second reader", MLP.replace("output y", "output y\nnode Relu h1 -> z\noutput z")),
    ("product is an output", MLP.replace("output y", "output y\noutput h1")),
])
def test_fuse_matmul_bias_declines(case, text):
    st, p = plan(text, L.GRAPH_FUSE_BIAS)
    assert st.get("fuse-matmul-bias", 0) == 1, case              # only the second layer folds
    assert "Add:h2" in p


def test_fuse_act_and_half_on_the_mlp():
    st, p = plan(MLP, F)
    assert st["fuse-matmul-bias"] == 2 and st["fuse-act"] == 2 and st["half-out"] == 1 and st["steps"] == 2
    l1, l2 = p["MatMul:h2"], p["MatMul:h5"]
    assert field(l1, "act") == str(L.ACT_GELU_ERF) and field(l2, "act") == str(L.ACT_RELU)
    assert field(p["ingot.Gelu:h3"], "pass") == "1" and field(p["Relu:y"], "pass") == "1"
    # layer 1's value (through the Gelu) is read only by layer 2's A: bf16; layer 2 feeds the graph output: f32
    assert field(l1, "half") == "1" and field(l1, "bf16_out") == "1"
    assert field(l2, "half") == "1" and field(l2, "bf16_out") == "0"


def test_fuse_act_without_half_keeps_f32():
    st, p = plan(MLP, L.GRAPH_FUSE_BIAS | L.GRAPH_FUSE_ACT)
    assert st["fuse-act"] == 2 and "half-out" not in st
    assert all(field(v, "half") == "0" and field(v, "bf16_out") == "0" for v in p.values())


@pytest.mark.parametrize("case,text,fused", [
    ("not fusable (HardSwish)", MLP.replace("node ingot.Gelu h2 -> h3", "node HardSwish@14 h2 -> h3"), 1),
    ("tanh Gelu fuses", MLP.replace("node ingot.Gelu h2 -> h3", "node Gelu@20 h2 -> h3 s:approximate=tanh"), 2),
    ("MatMul with its own gelu", MLP.replace("node MatMul x,W1 -> h1", "node MatMul x,W1 -> h1 s:ingot_act=gelu"),
     1),
    ("dynamic weight", MLP.replace("const W2 f32 3072,768", "input W2 f32 3072,768"), 1),
])
def test_fuse_act_rules(case, text, fused):
    st, _ = plan(text, L.GRAPH_FUSE_BIAS | L.GRAPH_FUSE_ACT)
    assert st.get("fuse-act", 0) == fused, case


def test_half_value_with_a_non_product_reader_stays_f32():
    text = MLP.replace("output y", "output y\nnode Relu h3 -> z\noutput z")
    st, p = plan(text, F)
    # h3 (layer 1's Gelu, still fused) now has a non-product reader too, so layer 1 stores f32
    assert field(p["MatMul:h2"], "bf16_out") == "0"
    assert st.get("half-out", 0) == 0


def test_parse_errors():
    with pytest.raises(IngotError, match="not defined before its use"):
        Graph(None, "input x f32 2,2\nnode Relu q -> y\noutput y")
    with pytest.raises(IngotError, match="defined twice"):
        Graph(None, "input x f32 2,2\nnode Relu x -> x\noutput x")
    with pytest.raises(IngotError, match="unknown dtype"):
        Graph(None, "input x f99 2,2")
    with pytest.raises(IngotError, match="no outputs"):
        Graph(None, "input x f32 2,2")
    with pytest.raises(IngotError, match="not produced by a node"):
        Graph(None, "input x f32 2,2\noutput x")
    g = Graph(None, MLP)
    g.compile(0)
    with pytest.raises(IngotError, match="already compiled"):
        g.compile(0)
    g.free()
