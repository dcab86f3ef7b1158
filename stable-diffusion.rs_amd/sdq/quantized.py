"""Weights quantized at rest, and the policy that decides which ones
(crates/sd-models/src/mlx/quantized.rs), over libsdq.

Only 2-D weights whose input width divides the group size are quantized;
norms, biases and embeddings stay dense (quantized.rs:28-35, 168-174).  The
dispatching `linear` sends a quantized name to `QuantizedArray.matmul` (the
HIP kernels) and a dense one to the dense `x @ w.T` (mod.rs:181-189), then adds
the bias after the matmul (quantized.rs:314-317).
"""
from __future__ import annotations

from typing import Callable, Dict, Optional, Protocol

GROUP_SIZE = 64   # quantized.rs:45-46
DEFAULT_BITS = 4  # quantized.rs:47-49


def sensitive(name: str) -> bool:
    """Layers held at 8 bits under the default policy (quantized.rs:110-117)."""
    return (
        "_mod.lin" in name
        or "modulation" in name
        or "_embedder" in name
        or name.startswith("img_in")
        or name.startswith("txt_in")
        or name.startswith("final_layer")
    )


def indexed(name: str) -> bool:
    """Tensors read by row rather than multiplied: never quantized
    (quantized.rs:131-152)."""
    return (
        name == "shared.weight"
        or "relative_attention_bias" in name
        or "_embedding.weight" in name
        or name.endswith("pos_embed")
        or "prd_embedding" in name
        or "positional_embedding" in name
        or name == "x_embedder.proj.weight"
        or name == "model.embed_tokens.weight"
        or name == "lm_head.weight"
    )


def mixed(bits: int) -> Callable[[str], int]:
    """The default policy (quantized.rs:156-166): indexed tensors dense (0),
    sensitive layers at 8 bits, everything else at `bits`."""

    def policy(name: str) -> int:
        if indexed(name):
            return 0
        if sensitive(name):
            return 8
        return bits

    return policy


def quantizable(shape) -> bool:
    """2-D with the input width a multiple of the group size (quantized.rs:172-174)."""
    return len(shape) == 2 and shape[1] % GROUP_SIZE == 0


class QuantizedWeights:
    """Two maps consulted by name (quantized.rs:51-86)."""

    def __init__(self, quantized: Optional[dict] = None, dense: Optional[dict] = None):
        self.quantized: Dict[str, "QuantizedArray"] = quantized or {}
        self.dense: Dict[str, "Array"] = dense or {}

    def resident_bytes(self) -> int:
        q = sum(a.resident_bytes() for a in self.quantized.values())
        d = sum(a.elem_count() * 4 for a in self.dense.values())
        return q + d

    def __len__(self) -> int:
        return len(self.quantized) + len(self.dense)

    def is_empty(self) -> bool:
        return len(self) == 0

    def contains_key(self, name: str) -> bool:
        return name in self.quantized or name in self.dense

    # WeightSource (quantized.rs:359-380)
    def linear(self, x, name: str, bias, s):
        return linear(x, name, bias, self, s)

    def dense_tensor(self, name: str):
        from . import Error

        if name in self.dense:
            return self.dense[name]
        if name in self.quantized:
            raise Error(
                f"sdq: {name} is quantised; reach it through `linear` rather than dequantising it"
            )
        raise Error(f"sdq: missing tensor {name}")

    def optional(self, name: str):
        return self.dense.get(name)


class WeightSource(Protocol):
    """Where a model's weights come from, dense or quantized (quantized.rs:320-339)."""

    def linear(self, x, name: str, bias, s): ...

    def dense_tensor(self, name: str): ...

    def optional(self, name: str): ...


class DenseWeights(dict):
    """`impl WeightSource for Weights` (quantized.rs:341-356): every tensor dense."""

    def linear(self, x, name: str, bias, s):
        from . import Error

        if name not in self:
            raise Error(f"sdq: missing tensor {name}")
        return dense_linear(x, self[name], bias, s)

    def dense_tensor(self, name: str):
        from . import Error

        if name not in self:
            raise Error(f"sdq: missing tensor {name}")
        return self[name]

    def optional(self, name: str):
        return self.get(name)


def dense_linear(x, w, b, s):
    """`x @ w.T + b`, the diffusers Linear (sd-models/src/mlx/mod.rs:181-189)."""
    y = x.matmul_nt(w, s)
    return y.add(b, s) if b is not None else y


def from_dense(w: dict, bits: int, s) -> QuantizedWeights:
    """quantized.rs:265-267: `from_dense_with(w, mixed(bits))`."""
    return from_dense_with(w, mixed(bits), s)


def from_dense_with(w: dict, bits_for: Callable[[str], int], s) -> QuantizedWeights:
    """Quantize a dense map (quantized.rs:273-291).  `bits_for` returns the
    width per tensor; 0 keeps it dense.  Each quantized weight is evaluated
    before the next, as the reference does to free its dense source."""
    from . import QuantizedArray, eval as sdq_eval

    quantized: Dict[str, QuantizedArray] = {}
    dense = {}
    for name, array in w.items():
        bits = bits_for(name)
        if bits >= 2 and quantizable(array.shape):
            q = QuantizedArray.quantize(array, GROUP_SIZE, bits, s)
            sdq_eval([q.weight, q.scales, q.biases])
            quantized[name] = q
        else:
            dense[name] = array.contiguous(s)
    return QuantizedWeights(quantized, dense)


def from_gguf(path, bits: int, s) -> QuantizedWeights:
    """Load a GGUF checkpoint, quantizing the large weights as they are read
    (quantized.rs:181-216).  Each tensor's raw blocks go to the device; a
    quantized one is decoded and quantized there in one kernel (the dense f32
    form is never written), a dense one is decoded to float32.  Each result is
    evaluated before the next tensor is read, as the reference does."""
    return _from_gguf(path, bits, lambda name: name, s, "")


def from_gguf_renamed(path, bits: int, rename: Callable[[str], Optional[str]], s) -> QuantizedWeights:
    """from_gguf with names translated (quantized.rs:225-258): `rename` maps a
    file name to the model's name, or None for a tensor the model skips."""
    return _from_gguf(path, bits, rename, s, " this model recognises")


def _from_gguf(path, bits: int, rename, s, what: str) -> QuantizedWeights:
    from . import Error, eval as sdq_eval
    from .gguf import Gguf

    quantized = {}
    dense = {}
    with Gguf.open(path) as g:
        for info in g.tensors:
            name = rename(info.name)
            if name is None:
                continue
            want = mixed(bits)(name)
            if want >= 2 and quantizable(info.shape):
                q = g.quantize(info, GROUP_SIZE, want, s)
                sdq_eval([q.weight, q.scales, q.biases])
                quantized[name] = q
            else:
                a = g.dequantize(info, s)
                a.eval()
                dense[name] = a
    if not quantized and not dense:
        raise Error(f"gguf: {path} carries no tensors{what}")
    return QuantizedWeights(quantized, dense)


def linear(x, name: str, bias, w: QuantizedWeights, s):
    """The dispatching linear (quantized.rs:298-318)."""
    from . import Error

    if name in w.quantized:
        y = w.quantized[name].matmul(x, s)
    else:
        if name not in w.dense:
            raise Error(f"sdq: {name} is in neither map")
        y = x.matmul_nt(w.dense[name], s)
    return y.add(bias, s) if bias is not None else y
