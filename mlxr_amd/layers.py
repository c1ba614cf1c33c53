"""Quantized Linear / MLP layers: the caller side of q_gemm_dequant.

Mirror of the C++ classes in include/mlxr_linear.h, which follow the reference's
core/graph/layers.h:59-94 (Linear: in_features, out_features, bias; forward(x) over
x [..., in_features] with M = batch * seq, layers.cpp:86-99) and MLP::forward
(layers.cpp:391-414: down(swish(gate(x)) * up(x))).  Weights are packed GGUF blocks on the
device; every computation runs in libmlxr_qgemm.so (torch supplies memory and streams).
"""
from . import qgemm
from .qgemm import BF16, F16, F32, PackedWeight, QGemmError


def _dt(torch, dtype):
    return {torch.float32: F32, torch.float16: F16, torch.bfloat16: BF16}[dtype]


def swiglu(gate, up, out=None, stream=None):
    """swish(gate) * up elementwise (mlxr_swiglu), in the dtype of gate."""
    torch = qgemm._torch()
    if gate.shape != up.shape or gate.dtype != up.dtype:
        raise QGemmError(-3, "gate and up must have the same shape and dtype")
    gate, up = gate.contiguous(), up.contiguous()
    out = torch.empty_like(gate) if out is None else out
    qgemm._check(qgemm.lib().mlxr_swiglu(gate.data_ptr(), up.data_ptr(), out.data_ptr(), gate.numel(), _dt(torch, gate.dtype),
                   qgemm._stream_ptr(stream)))
    return out


class Linear:
    """y = x W^T (+ b) with W [out_features, in_features] held as packed GGUF blocks."""

    def __init__(self, in_features, out_features, bias=False):
        if in_features <= 0 or out_features <= 0:
            raise QGemmError(-1, "Linear: features must be positive")
        self.in_features, self.out_features, self.has_bias = in_features, out_features, bias
        self.weight = None
        self.bias = None

    def load_weight(self, src, quant_type=None, name=None, device="cuda"):
        """src: GGUF block bytes (numpy/torch uint8) with quant_type, a PackedWeight, or a
        GGUFFile with the tensor name."""
        from .gguf import GGUFFile
        if isinstance(src, PackedWeight):
            pw = src
        elif isinstance(src, GGUFFile):
            info = src.find_tensor(name)
            if info is None:
                raise QGemmError(-1, f"GGUF tensor not found: {name}")
            if info.dimensions != [self.in_features, self.out_features]:
                raise QGemmError(-3, f"GGUF tensor {name} does not have dims {{in_features, out_features}}")
            pw = src.upload(name, device=device)
        else:
            pw = qgemm.pack_weights(src, self.out_features, self.in_features, quant_type, device=device)
        if (pw.N, pw.K) != (self.out_features, self.in_features):
            raise QGemmError(-3, "weight shape does not match [out_features, in_features]")
        self.weight = pw
        return self

    def set_bias(self, bias):
        if not self.has_bias:
            raise QGemmError(-1, "Linear was built without bias")
        if bias.dim() != 1 or bias.shape[0] != self.out_features:
            raise QGemmError(-3, "Bias shape must be [N]")
        self.bias = bias

    def forward(self, x, stream=None):
        if self.weight is None:
            raise QGemmError(-1, "Linear: weight not loaded")
        if self.has_bias and self.bias is None:
            raise QGemmError(-1, "Linear: bias not set")
        if x.dim() < 1 or x.shape[-1] != self.in_features:
            raise QGemmError(-3, "Input shape must be [..., in_features]")
        lead = x.shape[:-1]
        M = 1
        for d in lead:
            M *= int(d)
        x2 = x.reshape(M, self.in_features)
        y = qgemm.q_gemm_dequant(x2, self.weight, M, self.out_features, self.in_features, self.weight.qtype,
                                 bias=self.bias, stream=stream)
        return y.reshape(*lead, self.out_features)

    __call__ = forward


class MLP:
    """down(swish(gate(x)) * up(x)) through mlxr_qgemm_mlp: at M = 1 the whole block is one
    launch; above, the fused gate/up/gating launch and the down projection.  The layer holds
    the workspace (sync words, h, split-K partials)."""

    def __init__(self, hidden_size, intermediate_size):
        self.hidden_size, self.intermediate_size = hidden_size, intermediate_size
        self.gate_proj = Linear(hidden_size, intermediate_size)
        self.up_proj = Linear(hidden_size, intermediate_size)
        self.down_proj = Linear(intermediate_size, hidden_size)
        self._ws = None

    def forward(self, x, stream=None):
        if x.dim() < 1 or x.shape[-1] != self.hidden_size:
            raise QGemmError(-3, "Input shape must be [..., hidden_size]")
        lead = x.shape[:-1]
        x2 = x.reshape(-1, self.hidden_size)
        gw, uw, dw = self.gate_proj.weight, self.up_proj.weight, self.down_proj.weight
        if gw is None or uw is None or dw is None:
            raise QGemmError(-1, "MLP: weights not loaded")
        if (gw.qtype, gw.N) == (uw.qtype, uw.N):
            if self._ws is None:
                self._ws = qgemm.MlpWorkspace(x.device)
            y = qgemm.q_gemm_mlp(x2, gw, uw, dw, self._ws, stream=stream)
        else:
            g = self.gate_proj.forward(x2, stream=stream)
            u = self.up_proj.forward(x2, stream=stream)
            h = swiglu(g, u, out=g, stream=stream)
            y = self.down_proj.forward(h, stream=stream)
        return y.reshape(*lead, self.hidden_size)

    __call__ = forward
