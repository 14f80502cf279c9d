"""CPU: the dispatcher surface (registry, KernelDispatcher, wire format,
REST service, CLI) behaves like the reference's, with the hip entries
registered; kernel calls on CPU tensors fail loudly (no CPU fallback)."""
import base64
import json

import numpy as np
import pytest
import torch

from dsl_tool_amd import gemm as G
from dsl_tool_amd.dispatcher import KernelDispatcher, get_registry
from dsl_tool_amd.dispatcher import cli as CLI
from dsl_tool_amd.dispatcher import dispatcher as D
from dsl_tool_amd.dispatcher.registry import KernelRegistry

NAMES = {"gemm.bf16_gemm", "gemm.lora_fused_gemm", "gemm.fp8_gemm", "gemm.fp4_gemm", "gemm.grouped_gemm",
         "normalization.rmsnorm_quant", "activations.swiglu_quant", "moe.routed_grouped_gemm"}


def test_registry_holds_the_hip_entries():
    reg = get_registry()
    ks = reg.list_kernels()
    assert {k["kernel_name"] for k in ks} == NAMES
    assert all(k["backend"] == "hip" for k in ks)
    assert reg.get("GEMM.FP8_GEMM", "HIP").fn is G.fp8_gemm       # keys are case-insensitive
    assert reg.get("gemm.fp4_gemm", "hip").fn is G.fp4_gemm
    assert reg.get("gemm.grouped_gemm", "hip").fn is G.grouped_gemm
    assert reg.get("gemm.bf16_gemm", "hip").fn is G.bf16_gemm
    from dsl_tool_amd import fused as FU
    assert reg.get("normalization.rmsnorm_quant", "hip").fn is FU.rmsnorm_quant
    assert reg.get("activations.swiglu_quant", "hip").fn is FU.swiglu_quant
    assert "weight" in reg.get("normalization.rmsnorm_quant", "hip").input_schema
    assert reg.list_backends_for("gemm.fp8_gemm") == ["hip"]
    assert reg.get("gemm.fp8_gemm", "triton") is None
    assert get_registry() is reg


def test_register_and_file_loader(tmp_path):
    reg = KernelRegistry()
    f = tmp_path / "k.py"
    f.write_text("def my_kernel(x, **kw):\n    return x * 2\n")
    fn = reg._try_load_attr_from_file(str(f), "my_kernel")
    reg.register("Custom.Double", "Hip", fn, "x2", input_schema={"x": "Tensor"})
    e = reg.get("custom.double", "hip")
    assert e.kernel_name == "custom.double" and e.fn(3) == 6 and e.input_schema == {"x": "Tensor"}
    assert reg._try_load_attr_from_file(str(tmp_path / "missing.py"), "x") is None
    bad = tmp_path / "bad.py"
    bad.write_text("raise ImportError('nope')\n")
    assert reg._try_load_attr_from_file(str(bad), "x") is None


def test_dispatcher_resolve_errors_and_info():
    d = KernelDispatcher()
    with pytest.raises(KeyError, match="Unknown kernel"):
        d.kernel_info("gemm.nope", "hip")
    with pytest.raises(KeyError, match="Available backends: \\['hip'\\]"):
        d.kernel_info("gemm.fp8_gemm", "triton")
    info = d.kernel_info("gemm.fp4_gemm", "hip")
    assert info["kernel_name"] == "gemm.fp4_gemm" and "fmt" in info["input_schema"]
    assert "num_groups" in d.kernel_info("gemm.grouped_gemm", "hip")["input_schema"]
    assert d.list_backends("gemm.grouped_gemm") == ["hip"]


@pytest.mark.skipif(torch.cuda.is_available(), reason="checks the no-GPU behaviour")
def test_kernel_on_cpu_tensors_fails_loudly():
    d = KernelDispatcher()
    assert d.device == "cpu"
    with pytest.raises(RuntimeError, match=r"Kernel 'gemm.fp8_gemm' \[hip\] raised: .*GPU"):
        d.run_from_spec("gemm.fp8_gemm", "hip",
                        [{"shape": [4, 32], "dtype": "bf16"}, {"shape": [32, 8], "dtype": "bf16"}],
                        {"scale_a": 1.0})


def test_shim_validation_precedes_any_launch():
    a = torch.zeros(4, 32, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="K mismatch"):
        G.fp8_gemm(a, torch.zeros(16, 8, dtype=torch.bfloat16))
    with pytest.raises(ValueError, match="fp4 format"):
        G.fp4_gemm(a, torch.zeros(32, 8, dtype=torch.bfloat16), fmt="fp6")
    with pytest.raises(TypeError, match="num_groups"):
        G.grouped_gemm(a, torch.zeros(2, 32, 8, dtype=torch.bfloat16), 2.5)
    with pytest.raises(ValueError, match="offsets"):
        G.grouped_gemm(a, torch.zeros(2, 32, 8, dtype=torch.bfloat16),
                       torch.tensor([0, 4], dtype=torch.int32))


# ------------------------------------------------------------- wire format --
def _b64(arr: np.ndarray) -> str:
    return base64.b64encode(np.ascontiguousarray(arr).tobytes()).decode()


@pytest.mark.parametrize("dtype,np_dtype", [("float32", np.float32), ("int32", np.int32),
                                            ("uint8", np.uint8), ("int64", np.int64)])
def test_deserialize_serialize_round_trip(dtype, np_dtype):
    arr = (np.arange(24).reshape(4, 6) % 7).astype(np_dtype)
    t = D.deserialize_tensor({"shape": [4, 6], "dtype": dtype, "data": _b64(arr)}, device="cpu")
    assert np.array_equal(t.numpy(), arr)
    back = D.serialize_tensor(t)
    assert back["shape"] == [4, 6]
    got = np.frombuffer(base64.b64decode(back["data"]), dtype=np_dtype).reshape(4, 6)
    assert np.array_equal(got, arr)


def test_bf16_travels_as_fp32_values():
    vals = np.float32([[1.0, -2.5], [0.15625, 3.0]])
    t = D.deserialize_tensor({"shape": [2, 2], "dtype": "bf16", "data": _b64(vals)}, "cpu")
    assert t.dtype == torch.bfloat16 and np.array_equal(t.float().numpy(), vals)
    out = D.serialize_tensor(t)
    assert out["dtype"] == "bfloat16"
    assert np.array_equal(np.frombuffer(base64.b64decode(out["data"]), np.float32), vals.ravel())


def test_fp8_and_e8m0_raw_bytes_and_random_fill():
    codes = np.array([[0x38, 0x7E, 0xFE, 0x00]], np.uint8)        # 1.0, 448, -448, 0
    t = D.deserialize_tensor({"shape": [1, 4], "dtype": "fp8", "data": _b64(codes)}, "cpu")
    assert t.dtype == torch.float8_e4m3fn and t.float().tolist() == [[1.0, 448.0, -448.0, 0.0]]
    assert base64.b64decode(D.serialize_tensor(t)["data"]) == codes.tobytes()
    e8 = D.deserialize_tensor({"shape": [2], "dtype": "e8m0",
                               "data": _b64(np.uint8([127, 130]))}, "cpu")
    assert e8.float().tolist() == [1.0, 8.0]
    r = D.deserialize_tensor({"shape": [64, 64], "dtype": "fp8", "fill": "random"}, "cpu")
    assert r.dtype == torch.float8_e4m3fn and r.float().abs().max() > 0
    assert D.summarize_tensor(r)["numel"] == 4096


def test_fill_modes_and_bad_inputs():
    z = D.deserialize_tensor({"shape": [3], "dtype": "fp32", "fill": "zeros"}, "cpu")
    o = D.deserialize_tensor({"shape": [3], "dtype": "int32", "fill": "ones"}, "cpu")
    f = D.deserialize_tensor({"shape": [2, 2], "dtype": "fp16", "fill": 2.5}, "cpu")
    assert z.sum() == 0 and o.tolist() == [1, 1, 1] and (f == 2.5).all()
    with pytest.raises(ValueError, match="Unknown dtype"):
        D.deserialize_tensor({"shape": [1], "dtype": "fp6"}, "cpu")
    with pytest.raises(ValueError, match="elements"):
        D.deserialize_tensor({"shape": [3], "dtype": "uint8", "data": _b64(np.uint8([1, 2]))},
                             "cpu")


def test_dispatch_result_to_dict():
    r = D.DispatchResult(torch.ones(2, dtype=torch.bfloat16), "gemm.fp8_gemm", "hip", 1.23456,
                         "cpu")
    d = r.to_dict()
    assert d["elapsed_ms"] == 1.2346 and d["output"]["shape"] == [2]
    r2 = D.DispatchResult([torch.zeros(1), 5], "k", "hip", 0.0, "cpu")
    assert r2.to_dict()["output"][1] == 5


# -------------------------------------------------------------------- REST --
@pytest.fixture(scope="module")
def client():
    from fastapi.testclient import TestClient

    from dsl_tool_amd.dispatcher.api import app
    with TestClient(app) as c:
        yield c


def test_rest_discovery(client):
    assert client.get("/health").json() == {"status": "ok", "service": "kernel-dispatcher"}
    body = client.get("/api/v1/kernels").json()
    assert body["count"] == len(NAMES) and {k["kernel_name"] for k in body["kernels"]} == NAMES
    det = client.get("/api/v1/kernels/gemm.fp8_gemm", params={"backend": "hip"}).json()
    assert det["backends_available"] == ["hip"] and "scale_a" in det["input_schema"]
    assert client.get("/api/v1/kernels/gemm.nope", params={"backend": "hip"}).status_code == 404


def test_rest_run_error_mapping(client):
    req = {"kernel_name": "gemm.nope", "backend": "hip",
           "inputs": [{"shape": [4, 32], "dtype": "bf16"}]}
    r = client.post("/api/v1/kernels/run", json=req)
    assert r.status_code == 404 and r.json()["error"] == "kernel_not_found"
    req = {"kernel_name": "gemm.fp8_gemm", "backend": "triton", "inputs": []}
    r = client.post("/api/v1/kernels/run", json=req)
    assert r.status_code == 404 and "hip" in r.json()["detail"]
    req = {"kernel_name": "gemm.fp8_gemm", "backend": "hip",
           "inputs": [{"shape": [4, 32], "dtype": "bf16"}, {"shape": [16, 8], "dtype": "bf16"}]}
    r = client.post("/api/v1/kernels/run", json=req)
    assert r.status_code == 400 and r.json()["error"] == "kernel_dispatch_failed"
    # request validation (pydantic) rejects unknown backends / dtypes / shapes
    for bad in ({"kernel_name": "x", "backend": "opencl"},
                {"kernel_name": "x", "backend": "hip", "inputs": [{"shape": [2], "dtype": "fp6"}]},
                {"kernel_name": "x", "backend": "hip", "inputs": [{"shape": [0, 2]}]}):
        assert client.post("/api/v1/kernels/run", json=bad).status_code == 422


# --------------------------------------------------------------------- CLI --
def test_cli_list_and_info(capsys):
    assert CLI.main(["list"]) == 0
    listed = json.loads(capsys.readouterr().out)
    assert {k["kernel_name"] for k in listed} == NAMES
    assert CLI.main(["info", "--kernel", "gemm.grouped_gemm", "--backend", "hip"]) == 0
    assert json.loads(capsys.readouterr().out)["kernel_name"] == "gemm.grouped_gemm"


def test_cli_param_coercion():
    p = CLI.parse_params(["num_groups=8", "scale_a=0.5", "x=true", "fmt=nvfp4"])
    assert p == {"num_groups": 8, "scale_a": 0.5, "x": True, "fmt": "nvfp4"}
    with pytest.raises(ValueError):
        CLI.parse_params(["novalue"])


def test_out_dtype_names_map_to_torch_dtypes():
    """JSON scalar params carry dtypes as strings (dispatcher.py:285-294)."""
    import torch

    from dsl_tool_amd import gemm as G
    for name in ("float32", "fp32", "torch.float32", "FLOAT32", "float"):
        assert G._as_dtype(name) == torch.float32
    for name in ("bfloat16", "bf16", "torch.bfloat16"):
        assert G._as_dtype(name) == torch.bfloat16
    assert G._as_dtype(torch.float32) == torch.float32
    with pytest.raises(ValueError):
        G._as_dtype("int8")
    with pytest.raises(ValueError):
        G._out_code(torch.float16)


def test_caller_output_must_match_the_product():
    """`out=` is written through by the kernels (ldc = its row stride), so a
    wrong shape, dtype, device or column stride is refused before any launch."""
    cpu = torch.device("cpu")
    c = G._out_tensor(None, 3, 5, "bf16", cpu)
    assert c.shape == (3, 5) and c.dtype == torch.bfloat16
    out = torch.empty(3, 8)[:, :5]                       # padded rows: ldc 8 >= 5
    assert G._out_tensor(out, 3, 5, torch.bfloat16, cpu) is out
    bad = [torch.empty(3, 4), torch.empty(5, 3), torch.empty(15),
           torch.empty(3, 5, dtype=torch.float16),
           torch.empty(5, 3).t(),                        # column stride 3
           torch.empty(3, 10)[:, ::2]]                   # column stride 2
    for b in bad:
        with pytest.raises(ValueError):
            G._out_tensor(b, 3, 5, torch.float32, cpu)
    with pytest.raises(ValueError):
        G._out_tensor(torch.empty(3, 5), 3, 5, torch.float32, torch.device("cuda", 0))
    with pytest.raises(TypeError):
        G._out_tensor([[0.0] * 5] * 3, 3, 5, torch.float32, cpu)
    # empty products take any [0, n] / [m, 0] tensor of the right shape
    assert G._out_tensor(torch.empty(0, 5), 0, 5, torch.float32, cpu).shape == (0, 5)
