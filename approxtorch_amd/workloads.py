"""Models and seeded synthetic inputs of the measured configurations.

ResNet-18 (CIFAR style: 3x3 stem, no max-pool, [2,2,2,2] basic blocks) and
ResNet-50 (torchvision v1.5 layout: stride on the 3x3 conv of each
bottleneck) are defined here because torchvision is not part of this
environment; both are plain nn.Module trees that convert_model walks like any
user model.  LUT recipes follow BASELINE.json's configs:
  c2 trunc4     ((a*b) >> 4) << 4 over int8 operands
  c3/c4 perturbed  a*b + round(N(0, 0.02*|a*b| + 1)), clipped to int16
  c5 u16mask    (a*b) & ~63 over uint8 operands (uint16 range)
"""
import numpy as np
import torch
import torch.nn as nn
import torch.nn.functional as F


# ------------------------------------------------------------------- LUTs
def lut_exact_int8():
    a = np.arange(256) - 128
    return (a[:, None] * a[None, :]).astype(np.float32).reshape(-1)


def lut_trunc4():
    a = np.arange(256) - 128
    return (((a[:, None] * a[None, :]) >> 4) << 4).astype(np.float32).reshape(-1)


def lut_perturbed(seed=0):
    a = np.arange(256, dtype=np.int64) - 128
    p = a[:, None] * a[None, :]
    g = torch.Generator().manual_seed(seed)
    noise = torch.randn((256, 256), generator=g, dtype=torch.float64).numpy()
    e = np.rint(noise * (0.02 * np.abs(p) + 1))
    return np.clip(p + e, -32768, 32767).astype(np.float32).reshape(-1)


def lut_u16mask():
    v = np.arange(256, dtype=np.int64)
    return ((v[:, None] * v[None, :]) & ~63).astype(np.float32).reshape(-1)


def lre_tables(lut, qtype="int8"):
    from . import grad_lut
    ga, gb = grad_lut.lre(np.asarray(lut).reshape(256, 256), qtype)
    return torch.from_numpy(ga), torch.from_numpy(gb)


def date_tables(lut, half_ws=2):
    from . import grad_lut
    ga, gb = grad_lut.DATE(np.asarray(lut).reshape(256, 256), half_ws)
    return torch.from_numpy(ga.reshape(-1)), torch.from_numpy(gb.reshape(-1))


# ----------------------------------------------------------------- models
class BasicBlock(nn.Module):
    expansion = 1

    def __init__(self, inp, planes, stride=1):
        super().__init__()
        self.conv1 = nn.Conv2d(inp, planes, 3, stride, 1, bias=False)
        self.bn1 = nn.BatchNorm2d(planes)
        self.conv2 = nn.Conv2d(planes, planes, 3, 1, 1, bias=False)
        self.bn2 = nn.BatchNorm2d(planes)
        self.shortcut = nn.Sequential()
        if stride != 1 or inp != planes:
            self.shortcut = nn.Sequential(nn.Conv2d(inp, planes, 1, stride, bias=False),
                                          nn.BatchNorm2d(planes))

    def forward(self, x):
        out = F.relu(self.bn1(self.conv1(x)))
        out = self.bn2(self.conv2(out))
        return F.relu(out + self.shortcut(x))


class Bottleneck(nn.Module):
    expansion = 4

    def __init__(self, inp, planes, stride=1):
        super().__init__()
        self.conv1 = nn.Conv2d(inp, planes, 1, bias=False)
        self.bn1 = nn.BatchNorm2d(planes)
        self.conv2 = nn.Conv2d(planes, planes, 3, stride, 1, bias=False)
        self.bn2 = nn.BatchNorm2d(planes)
        self.conv3 = nn.Conv2d(planes, planes * 4, 1, bias=False)
        self.bn3 = nn.BatchNorm2d(planes * 4)
        self.downsample = None
        if stride != 1 or inp != planes * 4:
            self.downsample = nn.Sequential(nn.Conv2d(inp, planes * 4, 1, stride, bias=False),
                                            nn.BatchNorm2d(planes * 4))

    def forward(self, x):
        idt = x if self.downsample is None else self.downsample(x)
        out = F.relu(self.bn1(self.conv1(x)))
        out = F.relu(self.bn2(self.conv2(out)))
        out = self.bn3(self.conv3(out))
        return F.relu(out + idt)


class ResNet(nn.Module):
    def __init__(self, block, layers, num_classes, cifar_stem):
        super().__init__()
        self.inp = 64
        if cifar_stem:
            self.conv1 = nn.Conv2d(3, 64, 3, 1, 1, bias=False)
            self.pool = nn.Identity()
        else:
            self.conv1 = nn.Conv2d(3, 64, 7, 2, 3, bias=False)
            self.pool = nn.MaxPool2d(3, 2, 1)
        self.bn1 = nn.BatchNorm2d(64)
        self.layer1 = self._make(block, 64, layers[0], 1)
        self.layer2 = self._make(block, 128, layers[1], 2)
        self.layer3 = self._make(block, 256, layers[2], 2)
        self.layer4 = self._make(block, 512, layers[3], 2)
        self.fc = nn.Linear(512 * block.expansion, num_classes)

    def _make(self, block, planes, n, stride):
        mods = []
        for s in [stride] + [1] * (n - 1):
            mods.append(block(self.inp, planes, s))
            self.inp = planes * block.expansion
        return nn.Sequential(*mods)

    def forward(self, x):
        x = self.pool(F.relu(self.bn1(self.conv1(x))))
        x = self.layer4(self.layer3(self.layer2(self.layer1(x))))
        return self.fc(torch.flatten(F.adaptive_avg_pool2d(x, 1), 1))


def resnet18_cifar(num_classes=10):
    return ResNet(BasicBlock, [2, 2, 2, 2], num_classes, cifar_stem=True)


def resnet50(num_classes=1000):
    return ResNet(Bottleneck, [3, 4, 6, 3], num_classes, cifar_stem=False)


def conv_lut_macs(model, input_shape):
    """Sum over converted convs of N*OH*OW*O*K (the LUT-MACs of one forward)."""
    from .nn import Conv2d_int8, Conv2d_uint8
    total = [0]

    def hook(m, inp, out):
        n, o, oh, ow = out.shape
        k = m.in_channels // m.groups * m.kernel_size[0] * m.kernel_size[1]
        total[0] += n * oh * ow * o * k

    hs = [m.register_forward_hook(hook) for m in model.modules()
          if isinstance(m, (Conv2d_int8, Conv2d_uint8))]
    with torch.no_grad():
        was = model.training
        model.eval()
        model(torch.zeros(input_shape, device=next(model.parameters()).device))
        model.train(was)
    for h in hs:
        h.remove()
    return total[0]


# ------------------------------------------------------------ configs
CONFIGS = {
    "c2": dict(model="resnet18_cifar", batch=128, hw=32, classes=10, qtype="int8",
               grad="ste", weight_bits=8, lut="trunc4", momentum=0.1),
    "c4": dict(model="resnet50", batch=64, hw=224, classes=1000, qtype="int8",
               grad="lre", weight_bits=8, lut="perturbed", momentum=0.05),
    "c5": dict(model="resnet50", batch=128, hw=224, classes=1000, qtype="uint8",
               grad="custom", weight_bits=4, lut="u16mask", momentum=0.05),
}


def build_training_workload(name, device, batch=None, seed=0):
    """(model, optimizer, x, labels, cfg) of a training config, seeded."""
    from .convert_model import convert_model
    cfg = dict(CONFIGS[name])
    if batch is not None:
        cfg["batch"] = batch
    torch.manual_seed(seed)
    model = resnet18_cifar(cfg["classes"]) if cfg["model"] == "resnet18_cifar" \
        else resnet50(cfg["classes"])
    lut_np = {"trunc4": lut_trunc4, "perturbed": lut_perturbed,
              "u16mask": lut_u16mask}[cfg["lut"]]()
    lut = torch.from_numpy(lut_np).to(device)
    dx = dw = None
    if cfg["grad"] == "lre":
        dx, dw = (t.to(device) for t in lre_tables(lut_np, cfg["qtype"]))
    elif cfg["grad"] == "custom":
        dx, dw = (t.to(device) for t in date_tables(lut_np, 2))
    model = convert_model(model, lut, qtype=cfg["qtype"], grad=cfg["grad"], dx=dx, dw=dw,
                          scale_momentum=cfg["momentum"], weight_bits=cfg["weight_bits"])
    model = model.to(device).train()
    opt = torch.optim.SGD(model.parameters(), lr=0.01, momentum=0.9)
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(cfg["batch"], 3, cfg["hw"], cfg["hw"], generator=g).to(device)
    y = torch.randint(0, cfg["classes"], (cfg["batch"],), generator=g).to(device)
    return model, opt, x, y, cfg


def training_step(model, opt, x, y):
    opt.zero_grad(set_to_none=True)
    loss = F.cross_entropy(model(x), y)
    loss.backward()
    opt.step()
    return loss
