"""windlass_amd - MI355X (gfx950) quantized-matmul backend for Windlass.

Host-side mirror of the reference's operator interface for this path, over the C ABI of
libwindlass_hip.so (include/windlass_hip.h):

- ``GgmlType``                    enum GgmlType (src/Gguf.cs:19-25)
- ``Quants.CanDecode/CanDot``     src/Quants.cs:11-21, 56-65
- ``WeightView`` / ``Slice``      src/LayerStream.cs:15-35 (here: raw blocks resident in HBM)
- ``Transformer.MatMul``          src/Transformer.cs:483-537 (+ MatMulEach, :544-561)
- ``Transformer.SwiGlu``          src/Transformer.cs:241-251
- ``Transformer.Route``           src/Transformer.cs:315-340
- ``Transformer.MoeFfn``          src/Transformer.cs:259-294 (router logits given)
- ``Context.IntDot``              Transformer.IntDot (src/Transformer.cs:23), the integer branch
                                  of MatMul (src/Transformer.cs:504-524)
- ``FastMath``                    CanIntDot/NeedsK/Fits/Quantize (src/FastMath.cs:27-91)
- ``Stage`` / ``HostBuffer``      LayerStream's slots and their reads (src/LayerStream.cs:36-264), in HBM
- ``LayerDesc`` + wl_layer_dev    Transformer.Layer (src/Transformer.cs:177-232) on device-resident activations
- ``DeviceTransformer``           Transformer.Forward/Head (src/Transformer.cs:83-125) and the greedy
                                  loop (src/Engine.cs:356-360), every tensor resident in HBM
- ``DeviceBatch``                 Transformer.ForwardBatch (src/Transformer.cs:127-170) and BatchEngine's
                                  stacked step (src/BatchEngine.cs:127-173): KV slots, one pass per step
- ``gguf.GgufModelFile``          GgufModelFile (src/Gguf.cs:104-270); ``gguf.model_config`` and
                                  ``gguf.load_device_model``: ModelConfig.From and a file's model in HBM

Errors map to the reference's exception kinds: ``NotSupportedError`` (NotSupportedException),
``ShapeError`` (ArgumentException), ``ArgumentOutOfRangeError``, ``BackendError`` (device
failure). There is no CPU fallback: without the built library every call raises.
"""
from ._lib import (ArgumentOutOfRangeError, BackendError, NotSupportedError, ShapeError,
                   library_path, load)
from .backend import (Context, FastMath, GgmlType, Graph, HostBuffer, LayerDesc, QActs, Quants, Stage,
                      Transformer, WeightView, layout)
from .model import DeviceBatch, DeviceTransformer, ModelConfig, StageStream

__all__ = ["ArgumentOutOfRangeError", "BackendError", "NotSupportedError", "ShapeError",
           "library_path", "load", "Context", "FastMath", "GgmlType", "Graph", "HostBuffer", "LayerDesc", "QActs", "Quants", "Stage",
           "Transformer", "WeightView", "layout", "DeviceBatch", "DeviceTransformer", "ModelConfig", "StageStream"]
