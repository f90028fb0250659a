"""bitsandbytes-compatible NF4 surface backed by the HIP library.

bitsandbytes is not available for this ROCm build, so the drop-in keeps the
call signatures and QuantState fields that the reference's patch surface and
tests rely on (reference solution/kernels/nf4.py:140-168,
solution/nf4_patch.py:62-125, solution/tests/test_nf4.py:40-44,136-137,
solution/tests/test_lora.py:99-100, solution/tests/test_unpad.py:261-266):

  functional.quantize_4bit(A, blocksize=64, compress_statistics=True, quant_type="nf4")
      -> (packed uint8 [ceil(n/2), 1], QuantState)
  functional.dequantize_4bit(A, quant_state=None, absmax=None, out=None, blocksize=None,
                             quant_type="fp4")
  matmul_4bit(A, B, quant_state, out=None, bias=None)      (B = packed.t())
  nn.Params4bit(data, requires_grad=False, compress_statistics=True, quant_type="nf4")
  nn.Linear4bit(in, out, bias=True, compute_dtype=torch.float16,
                compress_statistics=True, quant_type="nf4")

Only the format on the reference's hot path is implemented: NF4, blocksize
64, double-quantized statistics (state2 blocksize 256, fp32), fp16 compute.
Anything else raises NotImplementedError -- there is no CPU path.
"""

import json
from types import SimpleNamespace

import torch

from . import _lib
from .kernels.nf4 import _validate_state, dequantize_nf4
from .kernels.nf4_gemm import NF4Linear


def dynamic_map_signed():
    """The 256-entry signed dynamic 8-bit code used for the second-level statistics.

    bitsandbytes create_dynamic_map(signed=True, max_exponent_bits=7,
    total_bits=8): for exponent i in 0..6, the 2**i midpoints of
    linspace(0.1, 1, 2**i + 1) scaled by 10**(i - 6), with both signs, plus
    0 and 1, sorted.  Format data; computed once per process.
    """
    global _DYNAMIC
    if _DYNAMIC is None:
        data = []
        for i in range(7):
            bounds = torch.linspace(0.1, 1.0, 2 ** i + 1, dtype=torch.float32)
            means = (bounds[:-1] + bounds[1:]) / 2.0
            scaled = (10.0 ** (i - 6)) * means
            data += scaled.tolist() + (-scaled).tolist()
        data += [0.0, 1.0]
        _DYNAMIC = torch.tensor(sorted(data), dtype=torch.float32)
    return _DYNAMIC


_DYNAMIC = None


def pack_dict_to_tensor(items):
    """The non-tensor items of a serialized QuantState as one uint8 tensor: the UTF-8
    bytes of ``json.dumps(items)`` (bitsandbytes' checkpoint format)."""
    return torch.tensor(list(json.dumps(items).encode("utf-8")), dtype=torch.uint8)


def unpack_tensor_to_dict(t):
    return json.loads(bytes(t.detach().cpu().numpy()).decode("utf-8"))


_QS_KEYS = ("absmax", "quant_map", "nested_absmax", "nested_quant_map", "quant_state",
            "quant_type", "blocksize", "dtype", "shape", "nested_blocksize", "nested_dtype",
            "nested_offset")


def _dtype_name(dtype):
    return str(dtype).split(".")[-1]


class QuantState:
    """NF4 quantization state with bitsandbytes' attribute names and checkpoint format.

    ``as_dict(packed=True)`` gives the tensors a ``Linear4bit`` state dict carries
    next to its packed weight -- absmax (uint8 block codes), quant_map (NF4
    table), nested_absmax / nested_quant_map (second-level statistics) and
    ``quant_state.bitsandbytes__nf4``, the JSON of the remaining fields packed
    into uint8 -- so safetensors checkpoints of bitsandbytes 0.50.2 and of this
    package load into each other; ``from_dict`` reads either form back.
    """

    valid_quant_types = ("fp4", "nf4")
    valid_qs_type_keys = tuple(f"bitsandbytes__{q}" for q in valid_quant_types)

    def __init__(self, absmax, shape=None, code=None, blocksize=None, quant_type=None,
                 dtype=None, offset=None, state2=None):
        self.absmax, self.shape, self.code = absmax, shape, code
        self.blocksize, self.quant_type, self.dtype = blocksize, quant_type, dtype
        self.offset, self.state2 = offset, state2
        self.nested = state2 is not None

    def to(self, device):
        device = torch.device(device)
        self.absmax = self.absmax.to(device)
        if self.offset is not None:
            self.offset = self.offset.to(device)
        if self.code is not None:
            self.code = self.code.to(device)
        if self.state2 is not None:
            self.state2.absmax = self.state2.absmax.to(device)
            self.state2.code = self.state2.code.to(device)
        return self

    def as_dict(self, packed=False):
        items = {"quant_type": self.quant_type, "absmax": self.absmax,
                 "blocksize": self.blocksize, "quant_map": self.code,
                 "dtype": _dtype_name(self.dtype), "shape": tuple(self.shape)}
        if self.nested:
            items.update({"nested_absmax": self.state2.absmax,
                          "nested_blocksize": self.state2.blocksize,
                          # its own storage: safetensors drops tensors that share one
                          "nested_quant_map": self.state2.code.clone(),
                          "nested_dtype": _dtype_name(self.state2.dtype),
                          "nested_offset": float(self.offset.reshape(-1)[0].item())})
        if not packed:
            return items
        out = {k: v for k, v in items.items() if isinstance(v, torch.Tensor)}
        rest = {k: v for k, v in items.items() if not isinstance(v, torch.Tensor)}
        out["quant_state.bitsandbytes__" + self.quant_type] = pack_dict_to_tensor(rest)
        return out

    @classmethod
    def from_dict(cls, qs_dict, device):
        """A QuantState from ``as_dict()`` output (packed or not; key prefixes allowed)."""
        qs_dict = dict(qs_dict)
        packed_keys = [k for k, v in qs_dict.items()
                       if "quant_state" in k and isinstance(v, torch.Tensor)]
        if not packed_keys and "quant_type" not in qs_dict:
            raise ValueError("expected packed or unpacked quant_state items, found neither")
        if packed_keys:
            if len(packed_keys) != 1 or packed_keys[0].split(".")[-1] not in \
                    cls.valid_qs_type_keys:
                raise ValueError(f"expected exactly one quant_state item ending in one of "
                                 f"{cls.valid_qs_type_keys}, found {packed_keys}")
            qs_dict.update(unpack_tensor_to_dict(qs_dict.pop(packed_keys[0])))
        qs_dict = {k.split(".")[-1]: v for k, v in qs_dict.items()}
        unknown = set(qs_dict) - set(_QS_KEYS)
        if unknown:
            raise ValueError(f"unknown quant_state items {sorted(unknown)}")
        device = torch.device(device)
        offset = state2 = None
        if "nested_absmax" in qs_dict:
            offset = torch.tensor(float(qs_dict["nested_offset"]), device=device)
            state2 = cls(absmax=qs_dict["nested_absmax"].to(device),
                         blocksize=qs_dict["nested_blocksize"],
                         code=qs_dict["nested_quant_map"].to(device),
                         dtype=getattr(torch, qs_dict["nested_dtype"]))
        shape = qs_dict["shape"]
        return cls(quant_type=qs_dict["quant_type"], absmax=qs_dict["absmax"].to(device),
                   blocksize=qs_dict["blocksize"], code=qs_dict["quant_map"].to(device),
                   dtype=getattr(torch, qs_dict["dtype"]),
                   shape=torch.Size(shape) if shape is not None else None,
                   offset=offset, state2=state2)


def quantize_4bit(A, absmax=None, out=None, blocksize=64, compress_statistics=True,
                  quant_type="nf4", quant_storage=torch.uint8):
    """Quantize a CUDA fp16/fp32 tensor to nested NF4 (ss_nf4_quantize)."""
    if quant_type != "nf4" or blocksize != 64 or not compress_statistics \
            or quant_storage != torch.uint8 or absmax is not None or out is not None:
        raise NotImplementedError("only nested NF4 / blocksize 64 / uint8 storage is supported")
    if not isinstance(A, torch.Tensor) or not A.is_cuda or A.dtype not in (torch.float16,
                                                                            torch.float32):
        raise ValueError("quantize_4bit expects a CUDA fp16/fp32 tensor")
    device = A.device
    flat = A.detach().contiguous().reshape(-1)
    n = flat.numel()
    if n == 0:
        raise ValueError("cannot quantize an empty tensor")
    blocks = -(-n // 64)
    packed = torch.empty((-(-n // 2), 1), device=device, dtype=torch.uint8)
    qabs = torch.empty(blocks, device=device, dtype=torch.uint8)
    absmax2 = torch.empty(-(-blocks // 256), device=device, dtype=torch.float32)
    code2 = dynamic_map_signed().to(device)
    offset = torch.empty(1, device=device, dtype=torch.float32)
    scratch = torch.empty(blocks, device=device, dtype=torch.float32)
    with torch.cuda.device(device):
        _lib.call("ss_nf4_quantize", flat.data_ptr(), _lib.dtype_code(flat.dtype), n,
                  packed.data_ptr(), qabs.data_ptr(), absmax2.data_ptr(), code2.data_ptr(),
                  offset.data_ptr(), scratch.data_ptr(), _lib.stream(device))
    state2 = QuantState(absmax2, code=code2, blocksize=256, dtype=torch.float32)
    nf4_code = torch.tensor(_nf4_table(), dtype=torch.float32, device=device)
    shape = tuple(A.shape) if A.ndim == 2 else (1, n)
    state = QuantState(qabs, shape=shape, code=nf4_code, blocksize=64, quant_type="nf4",
                       dtype=torch.float16, offset=offset, state2=state2)
    return packed, state


def _nf4_table():
    from .kernels.nf4 import NF4_VALUES

    return NF4_VALUES


def dequantize_4bit(A, quant_state=None, absmax=None, out=None, blocksize=None, quant_type="fp4"):
    """Decode a nested NF4 state (ss_nf4_dequant_nested); same view rule as bitsandbytes."""
    if quant_state is None:
        raise NotImplementedError("only dequantization from a QuantState is supported")
    shape = _validate_state(A, quant_state, torch.float16)
    if out is not None and (out.shape != shape or out.dtype != torch.float16
                            or out.device != A.device or not out.is_contiguous()):
        raise ValueError("out must be a contiguous fp16 tensor of quant_state.shape")
    return dequantize_nf4(A, quant_state, out=out)


def matmul_4bit(A, B, quant_state, out=None, bias=None):
    """A . dequant(B)^T (+bias) with autograd for A; B is the packed weight's .t() view."""
    if out is not None:
        raise NotImplementedError("out= is not supported")
    packed = B.t() if B.ndim == 2 and B.shape[0] == 1 else B
    return NF4Linear.apply(A, packed, quant_state, bias)


class Params4bit(torch.nn.Parameter):
    """Frozen NF4 weight: holds the fp16/fp32 data until moved to a GPU, then the packed bytes."""

    def __new__(cls, data=None, requires_grad=False, quant_state=None, blocksize=64,
                compress_statistics=True, quant_type="nf4", quant_storage=torch.uint8, **_):
        if data is None:
            data = torch.empty(0)
        self = torch.Tensor._make_subclass(cls, data, requires_grad)
        self.quant_state = quant_state
        self.blocksize, self.compress_statistics = blocksize, compress_statistics
        self.quant_type, self.quant_storage = quant_type, quant_storage
        return self

    @classmethod
    def from_prequantized(cls, data, quantized_stats, requires_grad=False, device="cuda",
                          module=None, **_):
        """A quantized weight from a checkpoint: packed codes + ``QuantState.as_dict`` items."""
        state = QuantState.from_dict(quantized_stats, device=device)
        self = cls(data.to(device), requires_grad=requires_grad, quant_state=state,
                   blocksize=state.blocksize, compress_statistics=state.nested,
                   quant_type=state.quant_type, quant_storage=data.dtype)
        if module is not None:
            module.quant_state = state
        return self

    def _quantize(self, device):
        packed, state = quantize_4bit(self.data.to(device), blocksize=self.blocksize,
                                      compress_statistics=self.compress_statistics,
                                      quant_type=self.quant_type)
        return Params4bit(packed, requires_grad=False, quant_state=state,
                          blocksize=self.blocksize, compress_statistics=self.compress_statistics,
                          quant_type=self.quant_type)

    def cuda(self, device=None, non_blocking=False):
        target = torch.device("cuda" if device is None else device)
        if self.quant_state is None:
            return self._quantize(target)
        return self

    def to(self, *args, **kwargs):
        device = kwargs.get("device")
        if device is None and args and isinstance(args[0], (str, torch.device)):
            device = args[0]
        if device is not None and torch.device(device).type == "cuda" and self.quant_state is None:
            return self._quantize(torch.device(device))
        return self


class Linear4bit(torch.nn.Linear):
    """bitsandbytes Linear4bit: NF4 frozen weight, fp16 compute, returns the input dtype."""

    def __init__(self, input_features, output_features, bias=True, compute_dtype=None,
                 compress_statistics=True, quant_type="nf4", quant_storage=torch.uint8,
                 device=None):
        super().__init__(input_features, output_features, bias, device)
        self.weight = Params4bit(self.weight.data, requires_grad=False,
                                 compress_statistics=compress_statistics, quant_type=quant_type,
                                 quant_storage=quant_storage)
        self.compute_dtype = compute_dtype
        self.compute_type_is_set = compute_dtype is not None
        self.quant_state = None
        if self.bias is not None:
            self.bias.requires_grad_(False)

    def _apply(self, fn, recurse=True):
        # Module.cuda()/.to()/.half() route through _apply.  The NF4 weight is
        # handled here: quantized once when it first reaches a GPU, and never
        # converted by fn afterwards (its bytes are the packed codes).
        weight = self._parameters.pop("weight")
        try:
            result = super()._apply(fn, recurse)
        finally:
            self._parameters["weight"] = weight
        probe = fn(torch.empty(0))
        if probe.is_cuda:
            if weight.quant_state is None:
                self.weight = weight._quantize(probe.device)
            elif weight.device != probe.device:
                raise NotImplementedError("moving a quantized Linear4bit between GPUs")
        return result

    def _save_to_state_dict(self, destination, prefix, keep_vars):
        super()._save_to_state_dict(destination, prefix, keep_vars)
        state = getattr(self.weight, "quant_state", None)
        if state is not None:
            for key, value in state.as_dict(packed=True).items():
                destination[prefix + "weight." + key] = value if keep_vars else value.detach()

    def _load_from_state_dict(self, state_dict, prefix, local_metadata, strict, missing_keys,
                              unexpected_keys, error_msgs):
        stats_prefix = prefix + "weight."
        stats = {k[len(stats_prefix):]: v for k, v in state_dict.items()
                 if k.startswith(stats_prefix)}
        packed = state_dict.get(prefix + "weight")
        if not stats or packed is None:
            super()._load_from_state_dict(state_dict, prefix, local_metadata, strict,
                                          missing_keys, unexpected_keys, error_msgs)
            return
        current = self.weight
        if packed.is_cuda:
            device = packed.device
        elif current.is_cuda:
            device = current.device
        else:
            device = torch.device("cuda", torch.cuda.current_device())
        self.weight = Params4bit.from_prequantized(packed, stats, device=device, module=self)
        rest = {k: v for k, v in state_dict.items()
                if k.startswith(prefix) and k != prefix + "weight" and not k.startswith(stats_prefix)}
        before = len(missing_keys)
        super()._load_from_state_dict(rest, prefix, local_metadata, strict, missing_keys,
                                      unexpected_keys, error_msgs)
        missing_keys[before:] = [k for k in missing_keys[before:] if k != prefix + "weight"]

    def forward(self, x):
        state = getattr(self.weight, "quant_state", None)
        if state is None:
            raise RuntimeError("Linear4bit weight is not quantized; move the module to a GPU")
        inp_dtype = x.dtype
        compute = self.compute_dtype or torch.float16
        if compute != torch.float16:
            raise NotImplementedError("only fp16 compute is supported")
        bias = None if self.bias is None else self.bias.to(torch.float16)
        x16 = x.to(torch.float16).contiguous()
        out = matmul_4bit(x16, self.weight.t(), state, bias=bias)
        return out.to(inp_dtype)


functional = SimpleNamespace(quantize_4bit=quantize_4bit, dequantize_4bit=dequantize_4bit,
                             QuantState=QuantState, pack_dict_to_tensor=pack_dict_to_tensor,
                             unpack_tensor_to_dict=unpack_tensor_to_dict)
nn = SimpleNamespace(Params4bit=Params4bit, Linear4bit=Linear4bit)

COMPAT_VERSION = "0.50.2+soupsuck_amd.compat"


def register_as_bitsandbytes():
    """Make ``import bitsandbytes`` (and ``.nn``, ``.functional``) resolve to this module.

    For images without bitsandbytes (this ROCm build): PEFT and user code that
    import bitsandbytes by name then get the NF4 surface above.  Returns False
    and changes nothing when a real bitsandbytes is importable or a module of
    that name is already loaded.  The version string is bitsandbytes' pinned
    0.50.2 with a local tag, so version checks parse it and the routes of
    soupsuck_amd.bnb_routes (built for the real 0.50.2 only) leave it alone.
    """
    import importlib.machinery
    import importlib.util
    import sys
    from types import ModuleType

    if "bitsandbytes" in sys.modules:
        return False
    try:
        if importlib.util.find_spec("bitsandbytes") is not None:
            return False
    except (ImportError, ValueError):
        return False
    package = ModuleType("bitsandbytes")
    package.__spec__ = importlib.machinery.ModuleSpec("bitsandbytes", None, is_package=True)
    package.__path__ = []
    package.__version__ = COMPAT_VERSION
    package.matmul_4bit = matmul_4bit
    children = {}
    for name, ns in (("nn", nn), ("functional", functional)):
        child = ModuleType(f"bitsandbytes.{name}")
        child.__spec__ = importlib.machinery.ModuleSpec(f"bitsandbytes.{name}", None)
        child.__dict__.update(vars(ns))
        setattr(package, name, child)
        children[f"bitsandbytes.{name}"] = child
    sys.modules["bitsandbytes"] = package
    sys.modules.update(children)
    return True
