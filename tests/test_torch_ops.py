"""The registered ops (workloadsuite_amd/torch_ops.py) that let torch.compile
trace the workload modules as single nodes -- the reference harness may wrap
a workload in torch.compile(fullgraph=False) (bench.py:185 of
ShouyangDong/WorkloadSuite).  CPU: the ops exist, their fake implementations
give the real outputs' shapes and dtypes, and a fake-mode trace of the module
holds one op node.  GPU: torch.compile(fullgraph=True) of both modules runs
and gives the eager module's bits."""

import pytest
import torch
from torch._subclasses.fake_tensor import FakeTensorMode
from torch.fx.experimental.proxy_tensor import make_fx

import workloadsuite_amd  # noqa: F401  (registers the ops)
from workloadsuite_amd import mamba_layer as ML
from workloadsuite_amd import mamba_ssd as MS

OPS = torch.ops.workloadsuite_amd


@pytest.mark.parametrize("final", [False, True])
def test_ssd_forward_fake_shapes(final):
    with FakeTensorMode():
        X = torch.empty(2, 512, 6, 64, dtype=torch.bfloat16)
        A = torch.empty(2, 512, 6)
        B = torch.empty(2, 512, 3, 128, dtype=torch.bfloat16)
        Y, f = OPS.ssd_forward(X, A, B, B, 256, None, None, final, torch.float32)
    assert Y.shape == X.shape and Y.dtype == X.dtype
    assert f.dtype == torch.float32 and f.shape == ((2, 6, 64, 128) if final else (0,))


def test_ssd_layer_fake_shape():
    with FakeTensorMode():
        x = torch.empty(2, 256, 4 * 64, dtype=torch.float16)
        B = torch.empty(2, 256, 2, 64, dtype=torch.float16)
        dt = torch.empty(2, 256, 4, dtype=torch.float16)
        w = torch.empty(4 * 64, 1, 4, dtype=torch.float16)
        hv = torch.empty(4, dtype=torch.float16)
        y = OPS.ssd_layer(x, x, B, B, dt, w, None, hv, torch.empty(4), None, 64, 4)
    assert y.shape == x.shape and y.dtype == x.dtype


def test_module_traces_to_one_op():
    model = MS.Model(2, 256, 4, 64, 32, block_len=64, n_groups=2)
    X = torch.randn(2, 256, 4, 64)
    params = {k: v.detach() for k, v in model.named_parameters()}
    gm = make_fx(lambda p, t: torch.func.functional_call(model, p, (t,)), tracing_mode="fake")(params, X)
    targets = [n.target for n in gm.graph.nodes if n.op == "call_function"]
    assert OPS.ssd_forward.default in targets


@pytest.mark.gpu
def test_compiled_ssd_model_equals_eager():
    torch.manual_seed(0)
    model = MS.Model(2, 512, 8, 64, 128, block_len=256, n_groups=2, dtype=torch.bfloat16,
                     return_final_state=True).cuda().eval()
    X = torch.randn(2, 512, 8, 64, device="cuda").to(torch.bfloat16)
    compiled = torch.compile(model, backend="eager", fullgraph=True)
    with torch.inference_mode():
        Ye, fe = model(X)
        Yc, fc = compiled(X)
    torch.cuda.synchronize()
    assert torch.equal(Ye, Yc) and torch.equal(fe, fc)


@pytest.mark.gpu
def test_compiled_layer_equals_eager():
    torch.manual_seed(0)
    layer = ML.SSDLayer(256, 4, 64, 64, 2, block_len=64, conv_kernel=4).cuda().eval()
    u = torch.randn(2, 512, 256, device="cuda", dtype=torch.float16)
    compiled = torch.compile(layer, backend="eager", fullgraph=True)
    with torch.inference_mode():
        ye = layer(u)
        yc = compiled(u)
    torch.cuda.synchronize()
    assert torch.equal(ye, yc)
