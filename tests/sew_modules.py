"""A module tree with the attribute names of the reference's sew_resnet18 (models/sewresnet.py:
26-66, 123-210): conv1 / bn1 / sn1 / maxpool / layer1..layer4 of blocks with conv1 and conv2
as containers holding `module = Sequential(conv, bn)`, sn1 / sn2 neurons, downsample =
Sequential(container, neuron), avgpool, fc, connect_f, neuron_type.  The neurons nest like the
reference's multi-step wrappers: MultiStepLIFNeuron / MultiStepIFNeuron keep their settings on a
single-step `neuron` member (models/neurons.py:187-231), the IF one without tau.  Test helper
for the front end: it holds the oracle's parameters under the same state_dict keys and carries
no forward."""
import torch
from torch import nn


class SeqToANN(nn.Module):
    def __init__(self, *mods):
        super().__init__()
        self.module = nn.Sequential(*mods)


class _LIFCore(nn.Module):
    def __init__(self, tau=2.0, v_threshold=1.0, v_reset=0.0):
        super().__init__()
        self.tau, self.v_threshold, self.v_reset = tau, v_threshold, v_reset


class _IFCore(nn.Module):
    def __init__(self, v_threshold=1.0, v_reset=0.0):
        super().__init__()
        self.v_threshold, self.v_reset = v_threshold, v_reset


class MultiStepLIFNeuron(nn.Module):
    def __init__(self, tau=2.0, v_threshold=1.0, v_reset=0.0):
        super().__init__()
        self.neuron = _LIFCore(tau, v_threshold, v_reset)


class MultiStepIFNeuron(nn.Module):
    def __init__(self, v_threshold=1.0, v_reset=0.0, **_ignored_tau):
        super().__init__()
        self.neuron = _IFCore(v_threshold, v_reset)


def Neuron(neuron_type="if", **kw):
    """The reference's choice (models/sewresnet.py:124): IF for "if", else LIF."""
    return MultiStepIFNeuron(**kw) if neuron_type == "if" else MultiStepLIFNeuron(**kw)


class Block(nn.Module):
    def __init__(self, cin, planes, stride, downsample, neuron_type, neuron_kw):
        super().__init__()
        self.conv1 = SeqToANN(nn.Conv2d(cin, planes, 3, stride, 1, bias=False), nn.BatchNorm2d(planes))
        self.sn1 = Neuron(neuron_type, **neuron_kw)
        self.conv2 = SeqToANN(nn.Conv2d(planes, planes, 3, 1, 1, bias=False), nn.BatchNorm2d(planes))
        self.sn2 = Neuron(neuron_type, **neuron_kw)
        self.downsample = downsample
        self.connect_f = "ADD"


class SEWResNet18Modules(nn.Module):
    def __init__(self, num_classes=100, in_channels=3, neuron_type="if", neuron_kw=None):
        super().__init__()
        kw = neuron_kw or {}
        self.connect_f = "ADD"
        self.neuron_type = neuron_type
        self.conv1 = nn.Conv2d(in_channels, 64, 7, 2, 3, bias=False)
        self.bn1 = nn.BatchNorm2d(64)
        self.sn1 = Neuron(neuron_type, **kw)
        self.maxpool = SeqToANN(nn.MaxPool2d(3, 2, 1))
        inplanes = 64
        for si, (planes, stride) in enumerate(((64, 1), (128, 2), (256, 2), (512, 2))):
            blocks = []
            for bi in range(2):
                s = stride if bi == 0 else 1
                ds = None
                if bi == 0 and (s != 1 or inplanes != planes):
                    ds = nn.Sequential(SeqToANN(nn.Conv2d(inplanes, planes, 1, s, bias=False), nn.BatchNorm2d(planes)),
                                       Neuron(neuron_type, **kw))
                blocks.append(Block(inplanes, planes, s, ds, neuron_type, kw))
                inplanes = planes
            setattr(self, f"layer{si + 1}", nn.Sequential(*blocks))
        self.avgpool = SeqToANN(nn.AdaptiveAvgPool2d((1, 1)))
        self.fc = nn.Linear(512, num_classes)

    @classmethod
    def from_params(cls, params: dict, **kw):
        m = cls(num_classes=params["fc.weight"].shape[0], in_channels=params["conv1.weight"].shape[1], **kw)
        sd = m.state_dict()
        missing = [k for k in sd if k not in params and not k.endswith("num_batches_tracked")]
        assert not missing, missing
        m.load_state_dict({k: params.get(k, sd[k]) for k in sd})
        return m.eval()
