"""Fixtures that pin the KNX3 graph semantics independently of this repository's writer and parser.

Run in the build container (it needs the reference repository, which the GPU machines do not have):

    python tests/golden/make_torch_golden.py /root/reference

For each small PyTorch model below it imports the reference's own exporter (tools/torch_graph.py, which writes
through tools/knx3.py), exports the model to .knx, runs the model in PyTorch (float32, eval mode) on a seeded input and
writes tests/golden/torch/<name>.knx and <name>.npz (x: input as PyTorch takes it, y: PyTorch's output).  The tests
then require the CPU oracle and the GPU forward of those files to reproduce PyTorch's outputs, which fixes what the
reference's files mean — attention input and weight order, convolution row order (ky, kx, ci), channels-first input
(layout 1), LSTM gate order, folded BatchNorm — without relying on this repository's reading of the format.
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
OUT = os.path.join(HERE, "torch")


class Encoder:
    """two TransformerEncoderLayers: pre-norm with GELU, then post-norm with ReLU (batch_first)"""

    @staticmethod
    def build(torch, nn):
        class M(nn.Module):
            def __init__(self):
                super().__init__()
                self.a = nn.TransformerEncoderLayer(32, 4, 64, dropout=0.0, activation="gelu", batch_first=True,
                                                    norm_first=True)
                self.b = nn.TransformerEncoderLayer(32, 4, 64, dropout=0.0, activation="relu", batch_first=True,
                                                    norm_first=False)

            def forward(self, x):
                return self.b(self.a(x))

        return M(), (10, 32)


class ConvNet:
    """channels-first image model: conv + BatchNorm (folded at export) + ReLU, strided grouped conv, max pool,
    pointwise conv, spatial mean, Linear"""

    @staticmethod
    def build(torch, nn):
        class M(nn.Module):
            def __init__(self):
                super().__init__()
                self.c1 = nn.Conv2d(3, 8, 3, padding=1)
                self.bn = nn.BatchNorm2d(8)
                self.c2 = nn.Conv2d(8, 12, 3, stride=2, padding=1, groups=4)
                self.pool = nn.MaxPool2d(2)
                self.c3 = nn.Conv2d(12, 12, 1)
                self.fc = nn.Linear(12, 6)

            def forward(self, x):
                h = torch.relu(self.bn(self.c1(x)))
                h = self.pool(torch.relu(self.c2(h)))
                return self.fc(self.c3(h).mean(dim=(2, 3)))

        m = M()
        with torch.no_grad():  # statistics away from (0, 1), so a wrong fold or channel order shows
            m.bn.running_mean.uniform_(-0.5, 0.5)
            m.bn.running_var.uniform_(0.5, 2.0)
            m.bn.weight.uniform_(0.5, 1.5)
            m.bn.bias.uniform_(-0.5, 0.5)
        return m, (3, 16, 16)


class BiLSTM:
    """bidirectional LSTM returning sequences, then a Linear on every timestep"""

    @staticmethod
    def build(torch, nn):
        class M(nn.Module):
            def __init__(self):
                super().__init__()
                self.rnn = nn.LSTM(6, 5, batch_first=True, bidirectional=True)
                self.fc = nn.Linear(10, 3)

            def forward(self, x):
                return self.fc(self.rnn(x)[0])

        return M(), (7, 6)


class Mlp:
    """Linear, LayerNorm, GELU, Linear, softmax"""

    @staticmethod
    def build(torch, nn):
        m = nn.Sequential(nn.Linear(20, 32), nn.LayerNorm(32), nn.GELU(), nn.Linear(32, 10), nn.Softmax(dim=-1))
        return m, (20,)


MODELS = {"encoder": (Encoder, None), "encoder_int8": (Encoder, "int8"), "convnet": (ConvNet, None),
          "bilstm": (BiLSTM, None), "mlp": (Mlp, None)}


def main(reference):
    sys.path.insert(0, os.path.join(reference, "tools"))
    import torch
    import torch.nn as nn
    from torch_graph import export_graph  # the reference's exporter

    os.makedirs(OUT, exist_ok=True)
    for i, (name, (spec, quantize)) in enumerate(sorted(MODELS.items())):
        torch.manual_seed(100 + i)
        model, shape = spec.build(torch, nn)
        model.eval()
        x = torch.randn((5,) + shape)
        with torch.no_grad():
            y = model(x).numpy()
        path = os.path.join(OUT, f"{name}.knx")
        layout = export_graph(model, path, shape, quantize)
        np.savez(os.path.join(OUT, f"{name}.npz"), x=x.numpy(), y=y, layout=np.int32(layout))
        print(f"{name}: {os.path.getsize(path)} bytes, layout {layout}, output {y.shape}")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
