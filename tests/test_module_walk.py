"""Module tree walk (minitorch_amd.module) on the CPU: the dotted keys and
their order, which tensors state_dict() and parameters() include, tied
weights and train/eval propagation -- the reference's Module contract
(module.py:5-118), restated here as expected lists.  No device memory: the
tensors are bare Tensor objects with only requires_grad set."""
from minitorch_amd.module import Module, Sequential
from minitorch_amd.tensor import Tensor


def _t(requires_grad=True):
    t = Tensor.__new__(Tensor)
    t.requires_grad = requires_grad
    return t


class Leaf(Module):
    def __init__(self):
        super().__init__()
        self.weight = _t()
        self.bias = _t()
        self.buffer = _t(requires_grad=False)  # not trainable: in neither list


class Tree(Module):
    def __init__(self):
        super().__init__()
        self.emb = _t()
        self.blocks = [Leaf(), Sequential(Leaf(), Leaf())]
        self.extra = [_t(), _t()]  # tensors held in a list: parameters() only
        self.head = Leaf()
        self.tied = self.head.weight  # the same tensor again: counted once


def test_state_keys_and_order():
    m = Tree()
    keys = [k for k, _ in m._named_state()]
    assert keys == ["emb",
                    "blocks.0.weight", "blocks.0.bias",
                    "blocks.1.layers.0.weight", "blocks.1.layers.0.bias",
                    "blocks.1.layers.1.weight", "blocks.1.layers.1.bias",
                    "head.weight", "head.bias",
                    "tied"]
    # the tied entry is the head's weight object under a second name
    st = dict(m._named_state())
    assert st["tied"] is st["head.weight"]


def test_parameters_order_lists_and_dedup():
    m = Tree()
    got = m.parameters()
    want = [m.emb,
            m.blocks[0].weight, m.blocks[0].bias,
            m.blocks[1].layers[0].weight, m.blocks[1].layers[0].bias,
            m.blocks[1].layers[1].weight, m.blocks[1].layers[1].bias,
            m.extra[0], m.extra[1],
            m.head.weight, m.head.bias]
    assert len(got) == len(want) and all(a is b for a, b in zip(got, want))


def test_train_eval_reach_every_module():
    m = Tree()
    mods = [m] + [v for kind, _, v, _ in m._walk() if kind == "module"]
    assert len(mods) == 1 + 1 + 1 + 2 + 1  # tree, blocks.0, blocks.1, its two leaves, head
    m.eval()
    assert not any(x._training for x in mods)
    m.train()
    assert all(x._training for x in mods)
