"""Host-side behaviour of the fp8 Linear mirror that needs no GPU."""
import pytest
import torch

from sr_dit import fp8_linear as fl


def test_constants_match_reference_module():
    assert fl.FP8_DTYPE is torch.float8_e4m3fn and fl.FP8_MAX == 448.0
    assert fl.TARGETS_ALL == ("self_attn.q", "self_attn.k", "self_attn.v", "self_attn.o",
                              "cross_attn.q", "cross_attn.k", "cross_attn.v", "cross_attn.o",
                              "ffn.0", "ffn.2")
    assert fl.TARGETS_FFN == ("ffn.0", "ffn.2")


def test_fp8_not_supported_on_cpu():
    assert fl.fp8_supported("cpu") is False
    if not torch.cuda.is_available():
        assert fl.fp8_supported() is False
        assert fl.prewarm_quantizer([(8, 128)]) == []


def test_convert_on_cpu_model_is_a_no_op():
    model = torch.nn.Module()
    model.blocks = torch.nn.ModuleList([torch.nn.Module()])
    model.blocks[0].ffn = torch.nn.Sequential(torch.nn.Linear(128, 128))
    assert fl.convert_linears_to_fp8(model) == []
    assert isinstance(model.blocks[0].ffn[0], torch.nn.Linear)


def test_fp8_linear_refuses_cpu_weight():
    with pytest.raises(RuntimeError, match="GPU"):
        fl.Fp8Linear(torch.zeros(16, 128))
    with pytest.raises(ValueError):
        fl.Fp8Linear(torch.zeros(16))


def test_quantiser_entry_points_refuse_cpu_tensors():
    with pytest.raises(RuntimeError):
        fl.quantize_rowwise(torch.zeros(4, 8))
    with pytest.raises(RuntimeError):
        fl.quantize_tensor(torch.zeros(4, 8))


def test_quantizer_shapes_closed_form():
    # fp8_linear.py:174-188: (M, dim) and (M, ffn_dim) per token count, then text shapes
    assert fl.quantizer_shapes([21600, 10368, 21600], 3072, 14336, [512]) == [
        (10368, 3072), (10368, 14336), (21600, 3072), (21600, 14336), (512, 3072)]


def test_block_index():
    assert fl._block_index("blocks.7.ffn.0") == 7
    assert fl._block_index("head.head") is None
