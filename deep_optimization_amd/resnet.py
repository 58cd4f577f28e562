"""ResNet-50, the CNN on which the compressed Conv / BatchNorm / ReLU layers run at model scale.

The reference applies its Controller to torchvision's ResNets (Activation_Compression/
test8.ipynb cell 2, ``models.resnet50``). torchvision is not a dependency of this library, so
this file defines the same architecture with torchvision's submodule names (``conv1``, ``bn1``,
``layer<k>.<i>.conv1..3 / bn1..3 / downsample``, ``fc``): a 7x7/2 stem with 3x3/2 max pooling,
bottleneck stages of 3, 4, 6 and 3 blocks (widths 64..512, expansion 4, stride on the 3x3
convolution), global average pooling and a linear classifier. Two differences: every ReLU call
site has its own module (``relu1..3`` in a block; torchvision calls one shared ``relu`` three
times, which would give three differently shaped activations one compression entry), and none
is in place. Weights use torchvision's initialisation (Kaiming-normal fan-out convolutions,
BatchNorm weight 1 and bias 0).
"""
from __future__ import annotations

from torch import nn


class Bottleneck(nn.Module):
    expansion = 4

    def __init__(self, inplanes: int, width: int, stride: int = 1, downsample: nn.Module | None = None):
        super().__init__()
        out = width * self.expansion
        self.conv1 = nn.Conv2d(inplanes, width, 1, bias=False)
        self.bn1 = nn.BatchNorm2d(width)
        self.relu1 = nn.ReLU()
        self.conv2 = nn.Conv2d(width, width, 3, stride=stride, padding=1, bias=False)
        self.bn2 = nn.BatchNorm2d(width)
        self.relu2 = nn.ReLU()
        self.conv3 = nn.Conv2d(width, out, 1, bias=False)
        self.bn3 = nn.BatchNorm2d(out)
        self.relu3 = nn.ReLU()
        self.downsample = downsample

    def forward(self, x):
        idt = x if self.downsample is None else self.downsample(x)
        y = self.relu1(self.bn1(self.conv1(x)))
        y = self.relu2(self.bn2(self.conv2(y)))
        y = self.bn3(self.conv3(y))
        return self.relu3(y + idt)


class ResNet(nn.Module):
    def __init__(self, layers=(3, 4, 6, 3), num_classes: int = 1000):
        super().__init__()
        self.inplanes = 64
        self.conv1 = nn.Conv2d(3, 64, 7, stride=2, padding=3, bias=False)
        self.bn1 = nn.BatchNorm2d(64)
        self.relu = nn.ReLU()
        self.maxpool = nn.MaxPool2d(3, stride=2, padding=1)
        self.layer1 = self._stage(64, layers[0], 1)
        self.layer2 = self._stage(128, layers[1], 2)
        self.layer3 = self._stage(256, layers[2], 2)
        self.layer4 = self._stage(512, layers[3], 2)
        self.avgpool = nn.AdaptiveAvgPool2d(1)
        self.fc = nn.Linear(512 * Bottleneck.expansion, num_classes)
        for m in self.modules():
            if isinstance(m, nn.Conv2d):
                nn.init.kaiming_normal_(m.weight, mode="fan_out", nonlinearity="relu")
            elif isinstance(m, nn.BatchNorm2d):
                nn.init.ones_(m.weight)
                nn.init.zeros_(m.bias)

    def _stage(self, width: int, blocks: int, stride: int) -> nn.Sequential:
        out = width * Bottleneck.expansion
        down = None
        if stride != 1 or self.inplanes != out:
            down = nn.Sequential(nn.Conv2d(self.inplanes, out, 1, stride=stride, bias=False), nn.BatchNorm2d(out))
        mods = [Bottleneck(self.inplanes, width, stride, down)]
        self.inplanes = out
        mods += [Bottleneck(out, width) for _ in range(1, blocks)]
        return nn.Sequential(*mods)

    def forward(self, x):
        x = self.maxpool(self.relu(self.bn1(self.conv1(x))))
        x = self.layer4(self.layer3(self.layer2(self.layer1(x))))
        return self.fc(self.avgpool(x).flatten(1))


def resnet50(num_classes: int = 1000) -> ResNet:
    return ResNet((3, 4, 6, 3), num_classes)


__all__ = ["ResNet", "Bottleneck", "resnet50"]
