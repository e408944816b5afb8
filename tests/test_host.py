"""Host-side behaviour of the Python drop-in surface (no GPU needed)."""

import pytest
import torch

import quantaweave_amd as qa
from quantaweave_amd import moe_kernels as mk


def small_config(**overrides):
    values = dict(vocab_size=32, hidden_size=16, layers=2, ffn_size=32, num_experts=6, top_k=2,
                  attention_heads=2, max_sequence_length=16, capacity_factor=0, min_expert_capacity=1)
    values.update(overrides)
    return qa.QuantaWeaveConfig(**values)


@pytest.mark.parametrize("bad", [dict(top_k=0), dict(top_k=7), dict(capacity_factor=-1), dict(min_expert_capacity=0),
                                 dict(overflow_policy="x"), dict(router_temperature=0), dict(hidden_size=15)])
def test_config_validation_mirrors_the_reference(bad):
    with pytest.raises(ValueError):
        small_config(**bad)


def test_capacity_follows_the_reference_formula():
    moe = qa.TopKMoE(small_config(capacity_factor=0.6, min_expert_capacity=2))
    assert moe.capacity(24) == 5
    moe.capacity_scale = 0.5
    assert moe.capacity(24) == 3
    moe.drop_overflow_tokens = False
    assert moe.capacity(24) == 48
    assert qa.TopKMoE(small_config()).capacity(10) == 20


def test_grouped_plan_bookkeeping():
    plan = mk.GroupedPlan([3, 0, 40], torch.device("cpu"))
    assert plan.tiles == 1 + 2 and plan.rows == 43
    assert plan.offsets.tolist() == [0, 3, 3, 43]
    assert mk.GroupedPlan([0, 0], torch.device("cpu")).tiles == 0
    with pytest.raises(ValueError):
        mk.GroupedPlan([1, -1], torch.device("cpu"))


def test_experts_support_grouped_accepts_plain_and_quantised_experts():
    moe = qa.TopKMoE(small_config())
    assert mk.experts_support_grouped(moe.experts)
    moe.experts[0].gate = torch.nn.Linear(16, 32, bias=True)
    assert not mk.experts_support_grouped(moe.experts)
    q = qa.QuantizedLinear(16, 32, bits=4)
    moe.experts[0].gate = q
    assert mk.experts_support_grouped(moe.experts)


def test_quantized_linear_geometry_and_errors():
    q = qa.QuantizedLinear(40, 24, bits=4, group_size=16)
    assert q.padded == 48 and q.qweight.shape == (24, 24) and q.qweight.dtype == torch.uint8
    assert q.scales.shape == (24, 3)
    q8 = qa.QuantizedLinear(40, 24, bits=8)
    assert q8.qweight.shape == (24, 40) and q8.scales.shape == (24, 1) and q8.qweight.dtype == torch.int8
    with pytest.raises(ValueError):
        qa.QuantizedLinear(8, 1, bits=4, group_size=7)
    with pytest.raises(ValueError):
        qa.QuantizedLinear(8, 1, bits=3)
    with pytest.raises(ValueError, match="bias"):
        qa.QuantizedLinear.from_linear(torch.nn.Linear(8, 4, bias=True))


def test_cpu_tensors_are_refused_not_computed():
    moe = qa.TopKMoE(small_config())
    with pytest.raises(RuntimeError, match="ROCm"):
        moe(torch.randn(1, 4, 16))
    with pytest.raises(RuntimeError):
        mk.grouped_swiglu(torch.randn(3, 16), moe.experts, [3, 0, 0, 0, 0, 0])


def test_kernel_selection_without_a_device():
    """tests/test_moe_kernels.py:137-143 of the reference: a CPU model falls
    back to the loop for "auto", keeps "loop", and refuses "triton"."""
    moe = qa.TopKMoE(small_config())
    with pytest.raises(ValueError):
        qa.set_moe_kernel(moe, "bogus")
    assert not mk.kernels_available(torch.device("cpu"))
    assert qa.set_moe_kernel(moe, "auto") == "loop" and qa.set_moe_kernel(moe, "loop") == "loop"
    assert moe.use_triton_kernels is False
    with pytest.raises(RuntimeError, match="CUDA"):
        qa.set_moe_kernel(moe, "triton")
    with pytest.raises(RuntimeError, match="CUDA"):
        qa.set_moe_kernel(moe, "hip")


def test_compute_dtype_rule():
    x = torch.randn(2, 3)
    assert mk.compute_dtype(x) == torch.float32
    with torch.autocast("cpu", dtype=torch.bfloat16):
        assert mk.compute_dtype(x) == torch.bfloat16


def test_decode_step_refuses_cpu_and_names_precisions():
    moe = qa.TopKMoE(small_config())
    with pytest.raises(RuntimeError, match="ROCm"):
        qa.MoEDecodeStep(moe, device=torch.device("cpu"))
    from quantaweave_amd.decode import precision_dtype
    # src/fast_decode.py:75-78
    assert precision_dtype(torch.device("cuda"), "auto") == torch.bfloat16
    assert precision_dtype(torch.device("cpu"), "auto") == torch.float32
    assert precision_dtype(torch.device("cuda"), "fp16") == torch.float16
    assert precision_dtype(torch.device("cuda"), "fp32") == torch.float32
    with pytest.raises(KeyError):
        precision_dtype(torch.device("cuda"), "fp8")


def test_expert_pack_currency_check_is_o1_and_sees_every_change():
    """The pack is re-stacked when the experts change; an armed pack checks
    one shared version counter, the registration generation and the first and
    last weight instead of every tensor."""
    import copy

    from quantaweave_amd.moe import packed_experts

    moe = qa.TopKMoE(small_config())
    ws = [getattr(e, n).weight for e in moe.experts for n in ("gate", "up", "down")]
    pack = packed_experts(moe, moe.experts)
    assert pack._token is not None and len(pack._reps) == 1         # one counter covers all 18 weights
    assert packed_experts(moe, moe.experts) is pack and pack.fast_current()
    # an optimizer step on one expert (in place): the shared counter moves
    opt = torch.optim.SGD([ws[7]], lr=0.1)
    ws[7].grad = torch.ones_like(ws[7])
    opt.step()
    assert not pack.fast_current()
    new = packed_experts(moe, moe.experts)
    assert new is not pack and torch.equal(new.up[2], ws[7].detach())
    # load_state_dict copies in place
    sd = {k: v.clone() + 1 for k, v in moe.state_dict().items()}
    moe.load_state_dict(sd)
    assert not new.fast_current()
    p2 = packed_experts(moe, moe.experts)
    assert torch.equal(p2.down[5], moe.experts[5].down.weight.detach())
    # replacing a projection module or a weight registers it: the generation moves
    moe.experts[3].up = torch.nn.Linear(16, 32, bias=False)
    assert not p2.fast_current()
    p3 = packed_experts(moe, moe.experts)
    assert torch.equal(p3.up[3], moe.experts[3].up.weight.detach())
    assert p3._token is not None and len(p3._reps) == 2            # the new weight has its own counter
    moe.experts[1].gate.weight = torch.nn.Parameter(torch.zeros(32, 16))
    assert not p3.fast_current()
    p4 = packed_experts(moe, moe.experts)
    assert p4.gate[1].abs().sum() == 0
    # a conversion of the whole module swaps every weight's data: the first and last storage move
    moe.half()
    assert not p4.fast_current()
    p5 = packed_experts(moe, moe.experts)
    assert p5.gate.dtype == torch.float16 and p5._token is not None
    # a copy re-checks everything on first use
    dup = copy.deepcopy(moe)
    assert dup._qw_pack._token is None
    moe.refresh_experts()
    assert "_qw_pack" not in moe.__dict__


def test_expert_weights_share_one_buffer_and_keep_their_values():
    torch.manual_seed(0)
    moe = qa.TopKMoE(small_config())
    ws = [getattr(e, n).weight for e in moe.experts for n in ("gate", "up", "down")]
    assert all(w.requires_grad and w.is_leaf for w in ws)
    base = ws[0].untyped_storage().data_ptr()
    assert all(w.untyped_storage().data_ptr() == base for w in ws)
    assert len({w.data_ptr() for w in ws}) == len(ws)
    # nn.Linear's init scale survives the move: |w| <= 1/sqrt(fan_in)
    assert max(float(w.detach().abs().max()) for w in ws[:2]) <= 16 ** -0.5
    assert set(dict(moe.named_parameters())) >= {"experts.0.gate.weight", "experts.5.down.weight"}
