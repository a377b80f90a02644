"""rdv_project_amd — MI355X-native (gfx950) implementation of rdv's small-network
hot path, behind rdv's own Python API.

    import rdv_project_amd as rdv
    m = rdv.linear(W0, b0, f16=True) >> rdv.relu >> rdv.linear(W1, b1, f16=True)
    y = m(rdv.wrap(x)).as_tensor('torch')

Public names follow the reference's curated surface (src/rdv/__init__.py:9-157)
for the parts this build implements: the node and generics machinery
(Node, Component, Struct, Main, Library, Generic, Generics, dispatch), the
value and pointer types (vec*/mat*, Type, Pointer, Buffer, FixArray, Deferred,
deferreds), the Map / Grid / TensorOperation families and their evaluators.  Compute runs only through the HIP library
(librdv_hip.so); there is no CPU fallback.
"""
from .core import (
    MemoryLocation,
    RDVObject,
    ensure_on_rdv,
    is_on_rdv,
    profiling,
    profiling_submit_times,
    reset_submit_times,
    set_synchronous,
    wrap,
)
from .maths import (
    BatchGridEvaluator,
    Composite,
    Constant,
    Grid,
    GridEvaluator,
    Identity,
    Map,
    MapEvaluator,
    Sensor,
    TensorOperation,
    TensorOpEvaluator,
    X,
    e,
    pi,
)
from .types import (
    Array,
    Buffer,
    Code,
    Component,
    CooperativeLibrary,
    Deferred,
    DeferredLibrary,
    FixArray,
    Generic,
    GenericParam,
    Generics,
    GridLibrary,
    Library,
    Main,
    MathLibrary,
    Node,
    Pointer,
    RandomLibrary,
    Single,
    Struct,
    Type,
    bvec2,
    bvec3,
    bvec4,
    deferreds,
    dispatch,
    ivec2,
    ivec3,
    ivec4,
    mat2,
    mat3,
    mat3x4,
    mat4,
    mat4x3,
    uvec2,
    uvec3,
    uvec4,
    vec2,
    vec3,
    vec4,
)
from ._conv import Winograd3x3Conv2d, winograd3x3_conv2d
from ._render import composite
from .grids import (
    Conv2D,
    Conv2dGrid,
    Downsample2x,
    MajorantGrid,
    TensorGrid,
    TensorGridBarrier,
    Upsample2x,
    barrier,
    conv2d,
    conv2d_o,
)
from ._train import mse_backward
from .rendering import (
    Cameras,
    EmissionAbsorption,
    EnvironmentSamplerTrait,
    EnvironmentTrait,
    ExtinctionTrait,
    MajorantTrait,
    RatiotrackingTransmittanceTrait,
    RaymarchingTransmittanceTrait,
    ScatteringAlbedoTrait,
    RatiotrackingTransmittance,
    RaymarchingTransmittance,
    VolumeProfile,
    VolumeProfileDDA,
    VoxelMajorantField,
)
from .nn import (
    ConcatTensorOp,
    Conv2DTensorOp,
    Conv2DTensorOpFast,
    Conv2DTensorOpSimple,
    Conv2DTensorOpSimple3x3,
    Conv2DTensorOpWindow3x3,
    Conv2DTensorOpWinograd3x3,
    Downsample2xTensorOp,
    Upsample2xTensorOp,
    DensityRGB,
    LinearTensorOp,
    LinearTensorOpFast,
    LinearTensorOpMine,
    LinearTensorOpSimple,
    LinearTensorOpSmall,
    ReLUTensorOp,
    FrequencyEncoding,
    Linear,
    LinearFast,
    ReLU,
    Sigmoid,
    Softplus,
    density_rgb,
    linear,
    relu,
    sigmoid,
    softplus,
)

__version__ = "0.1.0"
