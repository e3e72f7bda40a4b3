"""KAN feed-forward blocks and FFN replacement (kanforge/torch/transformer.py), host side:
structure of KANFFN / KATBlock, the FFN sites kanify finds in ViT-, GPT-2-, BERT- and
LLaMA-style modules, and the weights it moves. Forward parity runs on the GPU
(tests/test_gpu_layers.py)."""

import pytest
import torch
from torch import nn

import kanforge_amd as kf
from kanforge_amd.torch import GRKAN, KANFFN, KANLinear, KATBlock, from_mlp, kanify


class Conv1D(nn.Module):
    """GPT-2's projection: weight (in, out), y = x W + b."""

    def __init__(self, nf, nx):
        super().__init__()
        self.weight = nn.Parameter(torch.randn(nx, nf))
        self.bias = nn.Parameter(torch.randn(nf))

    def forward(self, x):
        return x @ self.weight + self.bias


class VitMLP(nn.Module):
    def __init__(self, d, h):
        super().__init__()
        self.fc1, self.act, self.fc2 = nn.Linear(d, h), nn.GELU(), nn.Linear(h, d)

    def forward(self, x):
        return self.fc2(self.act(self.fc1(x)))


class Gpt2MLP(nn.Module):
    def __init__(self, d, h):
        super().__init__()
        self.c_fc, self.act, self.c_proj = Conv1D(h, d), nn.GELU(approximate="tanh"), Conv1D(d, h)


class BertIntermediate(nn.Module):
    def __init__(self, d, h):
        super().__init__()
        self.dense, self.intermediate_act_fn = nn.Linear(d, h), nn.GELU()


class BertOutput(nn.Module):
    def __init__(self, d, h):
        super().__init__()
        self.dense = nn.Linear(h, d)


class BertLayer(nn.Module):
    def __init__(self, d, h):
        super().__init__()
        self.intermediate, self.output = BertIntermediate(d, h), BertOutput(d, h)


class LlamaMLP(nn.Module):
    def __init__(self, d, h):
        super().__init__()
        self.gate_proj, self.up_proj, self.down_proj, self.act_fn = nn.Linear(d, h), nn.Linear(d, h), nn.Linear(h, d), nn.SiLU()


def test_kanffn_and_katblock_structure():
    ffn = KANFFN(16, kind="grkan", groups=4)
    assert isinstance(ffn.fc1, GRKAN) and (ffn.fc1.in_features, ffn.fc1.out_features) == (16, 64)
    assert ffn.fc1.basis.init == "identity" and ffn.fc2.basis.init == "gelu"
    kan = KANFFN(16, 32, kind="kan", basis=kf.Chebyshev(6), base_activation=None)
    assert isinstance(kan.fc2, KANLinear) and kan.fc2.basis == kf.Chebyshev(6) and kan.fc2.base_weight is None
    blk = KATBlock(16, 4, mlp_ratio=2.0, groups=4)
    assert blk.ffn.fc1.out_features == 32 and isinstance(blk.attn, nn.MultiheadAttention)
    with pytest.raises(ValueError):
        KANFFN(8, kind="mlp")


def test_kanify_exact_moves_weights_and_activation():
    torch.manual_seed(0)
    model = nn.ModuleDict({"vit": VitMLP(8, 16), "gpt": Gpt2MLP(8, 16), "bert": BertLayer(8, 16), "llama": LlamaMLP(8, 16)})
    w_vit, w_gpt, w_bert, w_llama = (model["vit"].fc2.weight.clone(), model["gpt"].c_proj.weight.clone(),
                                     model["bert"].output.dense.weight.clone(), model["llama"].down_proj.weight.clone())
    done = kanify(model, "exact", basis=kf.BSpline(5, 3))
    assert sorted(done) == ["bert", "gpt", "llama", "vit"]
    vit, gpt, bert, llama = model["vit"], model["gpt"], model["bert"], model["llama"]
    assert isinstance(vit.act, nn.Identity) and isinstance(vit.fc2, KANLinear)
    assert isinstance(vit.fc2.base_activation, nn.GELU) and torch.equal(vit.fc2.base_weight, w_vit)
    assert torch.count_nonzero(vit.fc2.coef) == 0
    assert isinstance(gpt.c_fc, nn.Linear) and torch.equal(gpt.c_proj.base_weight, w_gpt.T)  # Conv1D turned around
    assert isinstance(bert.intermediate.intermediate_act_fn, nn.Identity) and torch.equal(bert.output.dense.base_weight, w_bert)
    assert isinstance(llama.down_proj, KANLinear) and torch.equal(llama.down_proj.base_weight, w_llama)
    with pytest.raises(TypeError):  # the rewritten sites hold KANLinear projections now
        kanify(model, "exact")


def test_kanify_grkan_transfers_weights():
    torch.manual_seed(1)
    model = nn.Sequential(VitMLP(8, 16))
    w1, b1 = model[0].fc1.weight.clone(), model[0].fc1.bias.clone()
    assert kanify(model, "grkan", groups=4) == ["0"]
    fc1, fc2 = model[0].fc1, model[0].fc2
    assert isinstance(fc1, GRKAN) and isinstance(fc2, GRKAN)
    assert fc1.basis.init == "identity" and fc2.basis.init == "gelu"
    torch.testing.assert_close(fc1.coef[..., 0], w1, rtol=0, atol=0)
    torch.testing.assert_close(fc1.bias, b1, rtol=0, atol=0)
    with pytest.raises(ValueError):
        kanify(nn.Sequential(VitMLP(4, 8)), "lora")


def test_from_mlp_pairs_activation_and_linear():
    torch.manual_seed(2)
    mlp = nn.Sequential(nn.Linear(4, 8), nn.Tanh(), nn.Linear(8, 3))
    net = from_mlp(mlp, kf.Chebyshev(4))
    assert isinstance(net[0], nn.Linear) and isinstance(net[1], KANLinear) and len(net) == 2
    assert isinstance(net[1].base_activation, nn.Tanh) and torch.equal(net[1].base_weight, mlp[2].weight)
    with pytest.raises(ValueError):
        from_mlp(nn.Sequential(nn.Tanh()))
