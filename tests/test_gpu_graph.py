"""HIP graph capture of the layers' eval-mode forward (torch.cuda.CUDAGraph).

The library launches on the capturing stream, takes its temporaries from
torch's allocator and issues no memset, copy or synchronisation of its own,
so a serving loop can capture a forward once and replay it.  Each case
replays the graph several times with the program's own eager work and
synchronisations in between (new input copied into the static input, an
eager forward of another input), and every replay equals the eager forward
of the same input bit for bit."""
import numpy as np
import pytest
import torch

import approxtorch_amd as at
from approxtorch_amd import workloads

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _int8_layer(k, s, p, O, wbits, grad):
    lut = torch.from_numpy(workloads.lut_perturbed(0)).to(DEV)
    kw = {}
    if grad == "lre":
        ga, gb = workloads.lre_tables(lut.cpu().numpy())
        kw = dict(dx=torch.as_tensor(ga).to(DEV), dw=torch.as_tensor(gb).to(DEV))
    return at.nn.Conv2d_int8(16, O, k, lut, grad=grad, bias=True, stride=s, padding=p,
                             weight_bits=wbits, **kw)


def _uint8_layer(k, s, p, O, wbits, grad):
    v = np.arange(256)
    lut = torch.from_numpy(((v[:, None] * v[None, :]) & ~63).astype(np.float32).reshape(-1))
    return at.nn.Conv2d_uint8(16, O, k, lut.to(DEV), grad=grad, bias=True, stride=s, padding=p,
                              weight_bits=wbits)


CASES = [
    ("int8 3x3 gather", _int8_layer, 3, 1, 1, 40, 8, "ste"),
    ("int8 1x1 rows", _int8_layer, 1, 1, 0, 72, 8, "ste"),
    ("int8 3x3 s2 lre", _int8_layer, 3, 2, 1, 24, 8, "lre"),
    ("int8 3x3 w4 matrix cores", _int8_layer, 3, 1, 1, 40, 4, "ste"),
    ("uint8 3x3 w4 matrix cores", _uint8_layer, 3, 1, 1, 40, 4, "ste"),
    ("uint8 3x3 w8", _uint8_layer, 3, 1, 1, 40, 8, "ste"),
]


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_eval_forward_graph_replays(case):
    _, make, k, s, p, O, wbits, grad = case
    torch.manual_seed(3)
    layer = make(k, s, p, O, wbits, grad).to(DEV)
    x0 = torch.randn(4, 16, 20, 20, device=DEV) + 0.3
    layer.train()
    with torch.no_grad():
        layer(x0)                                  # one EMA step sets the scales
    layer.eval()
    inputs = [torch.randn(4, 16, 20, 20, device=DEV) * (1 + i) + 0.2 * i for i in range(3)]
    with torch.no_grad():
        want = [layer(x).clone() for x in inputs]
        static_x = inputs[0].clone()
        layer(static_x)                            # warm-up on the capture's input
        torch.cuda.synchronize()
        s_cap = torch.cuda.Stream()
        s_cap.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s_cap):
            layer(static_x)                        # warm-up on the side stream as well
        torch.cuda.current_stream().wait_stream(s_cap)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            static_y = layer(static_x)
        for rep in range(2):
            for i, x in enumerate(inputs):
                static_x.copy_(x)
                graph.replay()
                got = static_y.clone()
                other = layer(inputs[(i + 1) % len(inputs)])     # eager work in between
                torch.cuda.synchronize()
                assert torch.equal(got, want[i]), (rep, i)
                assert torch.equal(other, want[(i + 1) % len(inputs)])


TRAIN_CASES = [
    ("int8 3x3 lre", _int8_layer, 3, 1, 1, 40, 8, "lre"),
    ("int8 1x1 ste", _int8_layer, 1, 1, 0, 72, 8, "ste"),
    ("uint8 3x3 w8 ste", _uint8_layer, 3, 1, 1, 40, 8, "ste"),
]


# make_graphed_callables warms the layer up on a side stream, where the
# parameters' gradient-accumulation nodes are created; torch then notes that
# the eager steps on the default stream feed them from another stream
@pytest.mark.filterwarnings("ignore:The AccumulateGrad node's stream")
@pytest.mark.parametrize("case", TRAIN_CASES, ids=[c[0] for c in TRAIN_CASES])
def test_train_step_graphed(case):
    """A training-mode layer under torch.cuda.make_graphed_callables (forward
    and backward each captured once, the EMA statistics included): over three
    steps with an SGD update of the weights in between, the outputs, the
    input, weight and bias gradients and the scale buffers equal an eager
    copy's bit for bit."""
    import copy
    _, make, k, s, p, O, wbits, grad = case
    torch.manual_seed(4)
    layer = make(k, s, p, O, wbits, grad).to(DEV).train()
    shape = (4, 16, 20, 20)
    with torch.no_grad():
        layer(torch.randn(shape, device=DEV) + 0.3)            # non-trivial scales
    state = {n: v.clone() for n, v in layer.state_dict().items()}
    eager = copy.deepcopy(layer)
    sample = torch.randn(shape, device=DEV, requires_grad=True)
    graphed = torch.cuda.make_graphed_callables(layer, (sample,))
    with torch.no_grad():                                       # undo the warm-up's EMA steps
        for n, v in layer.state_dict().items():
            v.copy_(state[n])
    layer.zero_grad(set_to_none=True)
    for step in range(3):
        x = torch.randn(shape, device=DEV) * (1 + step) + 0.1 * step
        xa, xb = x.clone().requires_grad_(), x.clone().requires_grad_()
        ya, yb = eager(xa), graphed(xb)
        g = torch.randn_like(ya)
        ya.backward(g)
        yb.backward(g)
        torch.cuda.synchronize()
        assert torch.equal(ya, yb), step
        assert torch.equal(xa.grad, xb.grad), step
        for (n, a), (_, b) in zip(eager.named_parameters(), layer.named_parameters()):
            assert torch.equal(a.grad, b.grad), (step, n)
        for (n, a), (_, b) in zip(eager.state_dict().items(), layer.state_dict().items()):
            assert torch.equal(a, b), (step, n)
        with torch.no_grad():
            for a, b in zip(eager.parameters(), layer.parameters()):
                a -= 0.05 * a.grad
                b -= 0.05 * b.grad
        eager.zero_grad(set_to_none=True)
        layer.zero_grad(set_to_none=True)
