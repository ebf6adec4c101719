"""The convnets of the benchmark configurations, built from plain torch.nn modules.

    plain_cnn()              PlainCNN: four conv3x3 (32, 64, 128, 256) + BatchNorm + ReLU + maxpool2x2 blocks in one
                             nn.Sequential (a fused stack), global average pool, linear 256 -> classes
    resnet18()               ResNet-18: 7x7/2 stem + BN + ReLU + 3x3/2 max pool, BasicBlocks [2, 2, 2, 2] at
                             64-128-256-512 channels with 1x1/2 projections, global average pool, linear 512 -> classes
    mobilenet_v3_small()     MobileNetV3-Small-style: inverted residuals with stride-1 depthwise 3x3 / 5x5, 1x1 expand /
                             project, hardswish, BatchNorm, squeeze-excite (adaptive average pool + linear)

Weights use Kaiming-normal initialization for convolutions (fan-in, ReLU gain), from torch's current RNG state.
These are the model definitions the benchmark configurations name; the reference's own variants differ in input
size, widths and classes (omarchy_mac_torch/models.py in the reference).
"""

import torch
from torch import nn


def _kaiming(model):
    for m in model.modules():
        if isinstance(m, nn.Conv2d):
            nn.init.kaiming_normal_(m.weight, mode="fan_in", nonlinearity="relu")
            if m.bias is not None:
                nn.init.zeros_(m.bias)
    return model


def plain_cnn(classes=10, in_ch=3, widths=(32, 64, 128, 256)):
    layers, c = [], in_ch
    for w in widths:
        layers += [nn.Conv2d(c, w, 3, padding=1, bias=False), nn.BatchNorm2d(w), nn.ReLU(), nn.MaxPool2d(2)]
        c = w
    return _kaiming(nn.Sequential(nn.Sequential(*layers), nn.AdaptiveAvgPool2d(1), nn.Flatten(),
                                  nn.Linear(c, classes)))


class BasicBlock(nn.Module):
    def __init__(self, cin, cout, stride):
        super().__init__()
        self.conv1 = nn.Conv2d(cin, cout, 3, stride, 1, bias=False)
        self.bn1 = nn.BatchNorm2d(cout)
        self.conv2 = nn.Conv2d(cout, cout, 3, 1, 1, bias=False)
        self.bn2 = nn.BatchNorm2d(cout)
        self.relu = nn.ReLU(inplace=True)
        self.down = None
        if stride != 1 or cin != cout:
            self.down = nn.Sequential(nn.Conv2d(cin, cout, 1, stride, bias=False), nn.BatchNorm2d(cout))

    def forward(self, x):
        y = self.relu(self.bn1(self.conv1(x)))
        y = self.bn2(self.conv2(y))
        return self.relu(y + (x if self.down is None else self.down(x)))


class ResNet18(nn.Module):
    def __init__(self, classes=1000, in_ch=3):
        super().__init__()
        self.stem = nn.Sequential(nn.Conv2d(in_ch, 64, 7, 2, 3, bias=False), nn.BatchNorm2d(64), nn.ReLU(inplace=True),
                                  nn.MaxPool2d(3, 2, 1))
        blocks, c = [], 64
        for w, s in ((64, 1), (128, 2), (256, 2), (512, 2)):
            blocks += [BasicBlock(c, w, s), BasicBlock(w, w, 1)]
            c = w
        self.blocks = nn.Sequential(*blocks)
        self.pool = nn.AdaptiveAvgPool2d(1)
        self.fc = nn.Linear(c, classes)
        _kaiming(self)

    def forward(self, x):
        return self.fc(torch.flatten(self.pool(self.blocks(self.stem(x))), 1))


def resnet18(classes=1000):
    return ResNet18(classes)


class SqueezeExcite(nn.Module):
    def __init__(self, c, r=4):
        super().__init__()
        self.pool = nn.AdaptiveAvgPool2d(1)
        self.fc1 = nn.Linear(c, max(8, c // r))
        self.fc2 = nn.Linear(max(8, c // r), c)

    def forward(self, x):
        s = torch.flatten(self.pool(x), 1)
        s = nn.functional.hardsigmoid(self.fc2(nn.functional.relu(self.fc1(s))))
        return x * s[:, :, None, None]


class InvertedResidual(nn.Module):
    def __init__(self, cin, exp, cout, k, se):
        super().__init__()
        self.expand = nn.Sequential(nn.Conv2d(cin, exp, 1, bias=False), nn.BatchNorm2d(exp), nn.Hardswish())
        self.dw = nn.Sequential(nn.Conv2d(exp, exp, k, 1, k // 2, groups=exp, bias=False), nn.BatchNorm2d(exp),
                                nn.Hardswish())
        self.se = SqueezeExcite(exp) if se else nn.Identity()
        self.project = nn.Sequential(nn.Conv2d(exp, cout, 1, bias=False), nn.BatchNorm2d(cout))
        self.residual = cin == cout

    def forward(self, x):
        y = self.project(self.se(self.dw(self.expand(x))))
        return x + y if self.residual else y


class MobileNetV3Small(nn.Module):
    """Stride-1 depthwise convs (the benchmark configuration); resolution drops by 2x2 max pools between stages."""

    def __init__(self, classes=1000, in_ch=3):
        super().__init__()
        self.stem = nn.Sequential(nn.Conv2d(in_ch, 16, 3, 2, 1, bias=False), nn.BatchNorm2d(16), nn.Hardswish())
        cfg = [  # (expansion, out, kernel, squeeze-excite, max pool after)
            (16, 16, 3, True, True), (72, 24, 3, False, True), (88, 24, 3, False, False),
            (96, 40, 5, True, True), (240, 40, 5, True, False), (120, 48, 5, True, False),
            (288, 96, 5, True, True), (576, 96, 5, True, False),
        ]
        layers, c = [], 16
        for exp, out, k, se, pool in cfg:
            layers.append(InvertedResidual(c, exp, out, k, se))
            if pool:
                layers.append(nn.MaxPool2d(2))
            c = out
        self.features = nn.Sequential(*layers)
        self.head = nn.Sequential(nn.Conv2d(c, 576, 1, bias=False), nn.BatchNorm2d(576), nn.Hardswish(),
                                  nn.AdaptiveAvgPool2d(1), nn.Flatten(), nn.Linear(576, classes))
        _kaiming(self)

    def forward(self, x):
        return self.head(self.features(self.stem(x)))


def mobilenet_v3_small(classes=1000):
    return MobileNetV3Small(classes)
