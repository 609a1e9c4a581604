"""Plan and catalog vocabulary of the FP8 path, with the MoE operation.

The reference's semantic plan and its kernel catalog are MoonBit, which this
image cannot compile. This module restates the parts a plan operation passes
through on its way to a launch, so that the MoE expert MLP (ExpertMlp, which
the reference has no operation for) has an executable definition beside the
operations it does have:

  OperationKind                 model/plan/operations.mbt:4-14, plus EXPERT_MLP
  operation shapes              model/plan/shapes.mbt:35-44, plus ExpertMlpShape
  kernel capability ids         model/plan/references.mbt:141-197, plus
                                expert_mlp = 11 (the next free id)
  PlanOperation constructors    model/plan/operations.mbt:31-159
  CatalogEntry legality         kernels/catalog/entry.mbt:17-228
  paged-v3 execution semantics  kernels/catalog/execution.mbt:136-175
  exact resolution              kernels/catalog/catalog.mbt:143-350

Every rule of the reference is kept as it is, with the same error kinds and
the same order of checks; the additions are one operation kind, one shape,
one capability and their legality rows: ExpertMlp takes an ExpertMlpShape and
the expert_mlp capability, and in a paged (v3) catalog it is stateless with
the StepCounts live input, as every operation other than rotary and attention
is. `fp8_entry` builds the catalog entry of an operation for this build's
code object (its family from the manifest, its workspace from the C ABI), and
`expert_mlp_steps` lists the launch steps an ExpertMlp binding runs.
"""
from __future__ import annotations

import enum
import hashlib
from dataclasses import dataclass, field


# --- plan vocabulary (model/plan) -------------------------------------------
class OperationKind(enum.Enum):
    EMBEDDING = "Embedding"
    RMS_NORM = "RmsNorm"
    QKV_PROJECTION = "QkvProjection"
    ROTARY_EMBEDDING = "RotaryEmbedding"
    CAUSAL_ATTENTION = "CausalAttention"
    OUTPUT_PROJECTION = "OutputProjection"
    RESIDUAL_ADD = "ResidualAdd"
    GATED_MLP = "GatedMlp"
    LANGUAGE_MODEL_HEAD = "LanguageModelHead"
    EXPERT_MLP = "ExpertMlp"  # added: routed expert MLP (top-k of E GatedMlps)


class PlanValidationError(ValueError):
    """kind: InvalidGraph / InvalidShape / InvalidWorkspaceBound /
    InvalidIdentifier (model/plan/errors.mbt); detail: the rule."""

    def __init__(self, kind: str, detail: str = ""):
        super().__init__(kind + (f"({detail})" if detail else ""))
        self.kind, self.detail = kind, detail


@dataclass(frozen=True)
class EmbeddingShape:
    vocabulary_size: int
    width: int


@dataclass(frozen=True)
class NormalizationShape:
    width: int
    epsilon: float


@dataclass(frozen=True)
class ProjectionShape:
    input_width: int
    output_width: int


@dataclass(frozen=True)
class RotaryShape:
    query_heads: int
    kv_heads: int
    head_dimension: int
    rope_theta: float


@dataclass(frozen=True)
class AttentionShape:
    query_heads: int
    kv_heads: int
    head_dimension: int


@dataclass(frozen=True)
class ElementwiseShape:
    width: int


@dataclass(frozen=True)
class GatedMlpShape:
    hidden_size: int
    intermediate_size: int


@dataclass(frozen=True)
class ExpertMlpShape:
    """Added. The routed MLP's dimensions, the same fields as the C ABI's
    routing descriptor (lunaflux_fp8_moe_descriptor): experts E, picks per
    token k, the routing rule (0: softmax over the k picked logits, 1:
    softmax over all E, keep the k picked), H, I, and the scale group (0 per
    token and per channel, 128 for 128-wide blocks)."""
    hidden_size: int
    intermediate_size: int
    experts: int
    top_k: int
    route_mode: int
    scale_group: int

    def __post_init__(self):
        if min(self.hidden_size, self.intermediate_size, self.experts, self.top_k) <= 0:
            raise PlanValidationError("InvalidShape", "PositiveDimension")
        if self.experts > 256 or self.top_k > self.experts or self.top_k > 16:
            raise PlanValidationError("InvalidShape", "ExpertRouting")
        if self.route_mode not in (0, 1):
            raise PlanValidationError("InvalidShape", "RouteMode")
        if self.hidden_size % 128 or self.intermediate_size % 128:
            raise PlanValidationError("InvalidShape", "TileWidth")
        if self.scale_group not in (0, 128) or (
                self.scale_group == 128 and max(self.hidden_size, self.intermediate_size) > 4096):
            raise PlanValidationError("InvalidShape", "ScaleGroup")


class Capability:
    """KernelCapabilityId stable ints (model/plan/references.mbt:141-197)."""
    EMBEDDING_LOOKUP = 1
    RMS_NORM = 2
    QKV_PROJECTION = 3
    ROTARY_EMBEDDING = 4
    CAUSAL_ATTENTION = 5
    DENSE_PROJECTION = 6
    RESIDUAL_ADD = 7
    GATED_MLP = 8
    POSITIONED_ROTARY_EMBEDDING = 9
    PAGED_CAUSAL_ATTENTION = 10
    EXPERT_MLP = 11  # added


class RuntimeInput(enum.Enum):
    STEP_COUNTS = "StepCounts"
    QUERY_POSITIONS = "QueryPositions"
    QUERY_ROW_OFFSETS = "QueryRowOffsets"
    SEQUENCE_LENGTHS = "SequenceLengths"
    PAGE_TABLE_OFFSETS = "PageTableOffsets"
    PAGE_TABLE_PAGE_INDICES = "PageTablePageIndices"


@dataclass(frozen=True)
class KvCacheReadWrite:
    layer: int


NO_PERSISTENT_STATE = None


@dataclass(frozen=True)
class Tensor:
    ref: int


@dataclass(frozen=True)
class Activation:
    ref: int


@dataclass(frozen=True)
class PlanOperation:
    id: int
    kind: OperationKind
    inputs: tuple
    outputs: tuple
    shape: object
    required_capability: int
    workspace_bytes: int
    kv_layer: int | None = None
    runtime_inputs: tuple = ()
    persistent_state: object = NO_PERSISTENT_STATE

    @staticmethod
    def _new(id, kind, inputs, outputs, shape, capability, workspace_bytes, kv_layer, runtime_inputs,
             persistent_state):
        # model/plan/operations.mbt:31-65
        if not inputs:
            raise PlanValidationError("InvalidGraph", "EmptyOperationInputs")
        if not outputs:
            raise PlanValidationError("InvalidGraph", "EmptyOperationOutputs")
        if workspace_bytes < 0:
            raise PlanValidationError("InvalidWorkspaceBound")
        return PlanOperation(id, kind, tuple(inputs), tuple(outputs), shape, capability, workspace_bytes,
                             kv_layer, tuple(runtime_inputs), persistent_state)

    @staticmethod
    def new_stateless(id, kind, inputs, outputs, shape, capability, workspace_bytes):
        # operations.mbt:74-97: rotary and attention are layered operations
        if kind in (OperationKind.ROTARY_EMBEDDING, OperationKind.CAUSAL_ATTENTION):
            raise PlanValidationError("InvalidGraph", "KvExecutionContract")
        return PlanOperation._new(id, kind, inputs, outputs, shape, capability, workspace_bytes, None, (),
                                  NO_PERSISTENT_STATE)

    @staticmethod
    def new_with_runtime_inputs(id, kind, inputs, outputs, shape, capability, workspace_bytes,
                                runtime_inputs):
        # operations.mbt:106-129
        if kind in (OperationKind.ROTARY_EMBEDDING, OperationKind.CAUSAL_ATTENTION) or not runtime_inputs:
            raise PlanValidationError("InvalidGraph", "KvExecutionContract")
        return PlanOperation._new(id, kind, inputs, outputs, shape, capability, workspace_bytes, None,
                                  runtime_inputs, NO_PERSISTENT_STATE)

    @staticmethod
    def expert_mlp(id, activation, router_logits, wg, wu, wd, descriptor, output, shape, workspace_bytes,
                   paged=True):
        """Added. The ExpertMlp node: inputs (activation, router logits [T,
        E] fp32, the expert weight stacks Wg, Wu [E, I, H] and Wd [E, H, I],
        the routing descriptor), one output activation; in a paged plan it
        consumes StepCounts (the live token count) like every stateless
        operation there."""
        inputs = (Activation(activation), Activation(router_logits), Tensor(wg), Tensor(wu), Tensor(wd),
                  Tensor(descriptor))
        if paged:
            return PlanOperation.new_with_runtime_inputs(id, OperationKind.EXPERT_MLP, inputs,
                                                         (Activation(output),), shape, Capability.EXPERT_MLP,
                                                         workspace_bytes, (RuntimeInput.STEP_COUNTS,))
        return PlanOperation.new_stateless(id, OperationKind.EXPERT_MLP, inputs, (Activation(output),), shape,
                                           Capability.EXPERT_MLP, workspace_bytes)


# --- catalog (kernels/catalog) -------------------------------------------------
class CatalogError(Exception):
    """kind: InvalidCatalog (rule in `rule`), UnsupportedExecutionContract,
    MissingKernel, IncompatibleTarget, IncompatibleImplementation,
    AmbiguousKernel, WorkspaceSizeOverflow, WorkspaceRequirementMismatch,
    WorkspaceLimitExceeded (operation id in `operation`)
    (kernels/catalog/errors.mbt:3-37)."""

    def __init__(self, kind: str, rule: str = "", operation: int | None = None):
        super().__init__(kind + (f"({rule})" if rule else "") + (f"({operation})" if operation is not None else ""))
        self.kind, self.rule, self.operation = kind, rule, operation


SEMANTIC_V1, SEMANTIC_V3 = 1, 3
CATALOG_V1, CATALOG_V3 = 1, 3


@dataclass(frozen=True)
class ContentAddressedAot:
    module_digest: str   # sha256 hex of the code object
    family_id: int


@dataclass(frozen=True)
class VendorBf16Gemm:
    """VendorBf16GemmImplicitHeuristicV1 (kept for its legality rules; no
    FP8 entry uses it)."""


@dataclass(frozen=True)
class ExecutionSemantics:
    kv_layer: int | None
    runtime_inputs: tuple
    persistent_state: object = NO_PERSISTENT_STATE
    kv_layout: object = None


@dataclass(frozen=True)
class DeviceTarget:
    compute_major: int
    compute_minor: int
    supports_bf16: bool = True
    supports_cublas_lt: bool = False


GFX950 = DeviceTarget(9, 5, True, False)

_SHAPE_OF = {
    OperationKind.EMBEDDING: EmbeddingShape,
    OperationKind.RMS_NORM: NormalizationShape,
    OperationKind.QKV_PROJECTION: ProjectionShape,
    OperationKind.OUTPUT_PROJECTION: ProjectionShape,
    OperationKind.LANGUAGE_MODEL_HEAD: ProjectionShape,
    OperationKind.ROTARY_EMBEDDING: RotaryShape,
    OperationKind.CAUSAL_ATTENTION: AttentionShape,
    OperationKind.RESIDUAL_ADD: ElementwiseShape,
    OperationKind.GATED_MLP: GatedMlpShape,
    OperationKind.EXPERT_MLP: ExpertMlpShape,
}


def operation_shape_is_legal(kind, shape) -> bool:
    # entry.mbt:54-70, plus (ExpertMlp, ExpertMlpShape)
    return isinstance(shape, _SHAPE_OF[kind])


def operation_capability_is_legal(semantic_version, kind, capability) -> bool:
    # entry.mbt:73-100, plus ExpertMlp -> expert_mlp
    v3 = semantic_version == SEMANTIC_V3
    expected = {
        OperationKind.EMBEDDING: Capability.EMBEDDING_LOOKUP,
        OperationKind.RMS_NORM: Capability.RMS_NORM,
        OperationKind.QKV_PROJECTION: Capability.QKV_PROJECTION,
        OperationKind.ROTARY_EMBEDDING: (Capability.POSITIONED_ROTARY_EMBEDDING if v3
                                         else Capability.ROTARY_EMBEDDING),
        OperationKind.CAUSAL_ATTENTION: (Capability.PAGED_CAUSAL_ATTENTION if v3
                                         else Capability.CAUSAL_ATTENTION),
        OperationKind.OUTPUT_PROJECTION: Capability.DENSE_PROJECTION,
        OperationKind.LANGUAGE_MODEL_HEAD: Capability.DENSE_PROJECTION,
        OperationKind.RESIDUAL_ADD: Capability.RESIDUAL_ADD,
        OperationKind.GATED_MLP: Capability.GATED_MLP,
        OperationKind.EXPERT_MLP: Capability.EXPERT_MLP,
    }[kind]
    return capability == expected


def _vendor_implementation_is_legal(kind, implementation) -> bool:
    # entry.mbt:29-38
    if isinstance(implementation, VendorBf16Gemm):
        return kind in (OperationKind.OUTPUT_PROJECTION, OperationKind.LANGUAGE_MODEL_HEAD)
    return True


def _vendor_workspace_is_legal(implementation, workspace_bytes, alignment) -> bool:
    # entry.mbt:41-51
    if isinstance(implementation, VendorBf16Gemm):
        return workspace_bytes == 0 or alignment == 256
    return True


def _is_power_of_two(v: int) -> bool:
    return v > 0 and v & (v - 1) == 0


def paged_semantics_are_legal(kind, s: ExecutionSemantics) -> bool:
    # execution.mbt:136-175: rotary and attention own layered roles; every
    # other kind, ExpertMlp included, is stateless with StepCounts only
    rt = RuntimeInput
    if kind == OperationKind.ROTARY_EMBEDDING:
        return (s.kv_layer is not None and s.runtime_inputs == (rt.STEP_COUNTS, rt.QUERY_POSITIONS)
                and s.persistent_state is NO_PERSISTENT_STATE and s.kv_layout is None)
    if kind == OperationKind.CAUSAL_ATTENTION:
        return (s.kv_layer is not None
                and s.runtime_inputs == (rt.STEP_COUNTS, rt.QUERY_POSITIONS, rt.QUERY_ROW_OFFSETS,
                                         rt.SEQUENCE_LENGTHS, rt.PAGE_TABLE_OFFSETS,
                                         rt.PAGE_TABLE_PAGE_INDICES)
                and s.persistent_state == KvCacheReadWrite(s.kv_layer) and s.kv_layout is not None)
    return (s.kv_layer is None and s.runtime_inputs == (rt.STEP_COUNTS,)
            and s.persistent_state is NO_PERSISTENT_STATE and s.kv_layout is None)


@dataclass(frozen=True)
class CatalogEntry:
    semantic_version: int
    operation_kind: OperationKind
    operation_shape: object
    capability: int
    compute_major: int
    compute_minor: int
    implementation: object
    workspace_bytes: int
    workspace_alignment: int
    execution_semantics: ExecutionSemantics | None = None

    @staticmethod
    def _common(kind, shape, capability, semantic_version, compute_major, compute_minor, workspace_bytes,
                workspace_alignment):
        if compute_major <= 0 or compute_minor < 0:
            raise CatalogError("InvalidCatalog", "InvalidComputeCapability")
        if workspace_bytes < 0:
            raise CatalogError("InvalidCatalog", "InvalidWorkspaceBytes")
        if not _is_power_of_two(workspace_alignment) or workspace_alignment > 65536:
            raise CatalogError("InvalidCatalog", "InvalidWorkspaceAlignment")
        if not operation_shape_is_legal(kind, shape):
            raise CatalogError("InvalidCatalog", "OperationShapeMismatch")
        if not operation_capability_is_legal(semantic_version, kind, capability):
            raise CatalogError("InvalidCatalog", "OperationCapabilityMismatch")

    @staticmethod
    def new(kind, shape, capability, compute_major, compute_minor, implementation, workspace_bytes,
            workspace_alignment, semantic_version=SEMANTIC_V1):
        # entry.mbt:103-147
        if semantic_version != SEMANTIC_V1:
            raise CatalogError("InvalidCatalog", "UnsupportedSemanticVersion")
        CatalogEntry._common(kind, shape, capability, semantic_version, compute_major, compute_minor,
                             workspace_bytes, workspace_alignment)
        if not _vendor_implementation_is_legal(kind, implementation):
            raise CatalogError("InvalidCatalog", "InvalidVendorImplementationKind")
        if not _vendor_workspace_is_legal(implementation, workspace_bytes, workspace_alignment):
            raise CatalogError("InvalidCatalog", "InvalidWorkspaceAlignment")
        return CatalogEntry(SEMANTIC_V1, kind, shape, capability, compute_major, compute_minor, implementation,
                            workspace_bytes, workspace_alignment, None)

    @staticmethod
    def new_paged_v3(kind, shape, capability, execution_semantics, compute_major, compute_minor,
                     implementation, workspace_bytes, workspace_alignment):
        # entry.mbt:155-206
        CatalogEntry._common(kind, shape, capability, SEMANTIC_V3, compute_major, compute_minor,
                             workspace_bytes, workspace_alignment)
        if not paged_semantics_are_legal(kind, execution_semantics):
            raise CatalogError("InvalidCatalog", "InvalidExecutionSemantics")
        if isinstance(implementation, VendorBf16Gemm):
            raise CatalogError("InvalidCatalog", "InvalidVendorImplementationKind")
        if not _vendor_implementation_is_legal(kind, implementation):
            raise CatalogError("InvalidCatalog", "InvalidVendorImplementationKind")
        if not _vendor_workspace_is_legal(implementation, workspace_bytes, workspace_alignment):
            raise CatalogError("InvalidCatalog", "InvalidWorkspaceAlignment")
        return CatalogEntry(SEMANTIC_V3, kind, shape, capability, compute_major, compute_minor, implementation,
                            workspace_bytes, workspace_alignment, execution_semantics)


@dataclass(frozen=True)
class KernelBinding:
    operation_id: int
    capability: int
    semantic_version: int
    execution_semantics: ExecutionSemantics | None
    implementation: object
    workspace_bytes: int
    workspace_alignment: int


@dataclass
class KernelCatalog:
    version: int
    entries: list = field(default_factory=list)

    def __post_init__(self):
        # catalog.mbt:84-129 (the family-consistency rules need the whole
        # manifest and are applied by the engine; the version rules here)
        if self.version not in (CATALOG_V1, CATALOG_V3):
            raise CatalogError("InvalidCatalog", "UnsupportedCatalogVersion")
        if not self.entries:
            raise CatalogError("InvalidCatalog", "EmptyCatalog")
        want = SEMANTIC_V1 if self.version == CATALOG_V1 else SEMANTIC_V3
        if any(e.semantic_version != want for e in self.entries):
            raise CatalogError("InvalidCatalog", "CatalogSemanticVersionMismatch")

    def _semantic_match(self, e: CatalogEntry, op: PlanOperation) -> bool:
        # catalog.mbt:143-175 (without the KV layout, which no FP8 entry has)
        if e.execution_semantics is None:
            execution = not op.runtime_inputs and op.persistent_state is NO_PERSISTENT_STATE
        else:
            s = e.execution_semantics
            execution = (s.kv_layer == op.kv_layer and s.persistent_state == op.persistent_state
                         and s.runtime_inputs == op.runtime_inputs)
        return (execution and e.operation_kind == op.kind and e.operation_shape == op.shape
                and e.capability == op.required_capability)

    def select_entry(self, op: PlanOperation, target: DeviceTarget) -> CatalogEntry:
        # catalog.mbt:215-250: missing, then target, then implementation,
        # then ambiguity
        semantic = [e for e in self.entries if self._semantic_match(e, op)]
        architecture = [e for e in semantic
                        if (e.compute_major, e.compute_minor) == (target.compute_major, target.compute_minor)]
        compatible = [e for e in architecture if target.supports_bf16 and (
            not isinstance(e.implementation, VendorBf16Gemm) or target.supports_cublas_lt)]
        if not semantic:
            raise CatalogError("MissingKernel", operation=op.id)
        if not architecture:
            raise CatalogError("IncompatibleTarget", operation=op.id)
        if not compatible:
            raise CatalogError("IncompatibleImplementation", operation=op.id)
        if len(compatible) != 1:
            raise CatalogError("AmbiguousKernel", operation=op.id)
        return compatible[0]

    def resolve(self, operations, target: DeviceTarget, workspace_limit: int) -> list:
        """Every operation bound exactly once (catalog.mbt:296-350): the
        entry's workspace rounded up to its alignment must cover the
        operation's and stay within the plan's limit."""
        bindings = []
        for op in operations:
            e = self.select_entry(op, target)
            rem = e.workspace_bytes % e.workspace_alignment
            required = e.workspace_bytes + (e.workspace_alignment - rem if rem else 0)
            if required > (1 << 63) - 1:
                raise CatalogError("WorkspaceSizeOverflow", operation=op.id)
            if required < op.workspace_bytes:
                raise CatalogError("WorkspaceRequirementMismatch", operation=op.id)
            if required > workspace_limit:
                raise CatalogError("WorkspaceLimitExceeded", operation=op.id)
            bindings.append(KernelBinding(op.id, op.required_capability, e.semantic_version,
                                          e.execution_semantics, e.implementation, required,
                                          e.workspace_alignment))
        return bindings


# --- this build's entries ------------------------------------------------------
def code_object_digest() -> str:
    from . import _abi
    return hashlib.sha256(_abi.code_object_bytes()).hexdigest()


def _descriptor(shape: ExpertMlpShape):
    from . import moe
    return moe.moe_descriptor(shape.experts, shape.top_k, shape.route_mode, shape.hidden_size,
                              shape.intermediate_size, shape.scale_group)


def expert_mlp_steps(shape: ExpertMlpShape, max_tokens: int) -> list:
    """The launch steps of an ExpertMlp binding for a profile: (step entry,
    symbol, grid, block), steps with no launch left out. All of them belong
    to the MoE family of the manifest; they run in order on one stream and
    share one workspace. (The reference binds one entry point per dense
    operation; ExpertMlp has no reference contract, and its routing and
    sort steps must finish before the grouped GEMMs can size their grids
    from the routed counts.)"""
    from . import _abi, moe
    desc = _descriptor(shape)
    out = []
    for entry in (_abi.MOE_ROUTE, _abi.MOE_SORT_COUNT, _abi.MOE_SORT, _abi.MOE_QUANT_TOKENS, _abi.MOE_GATE_UP,
                  _abi.MOE_QUANT_HIDDEN, _abi.MOE_DOWN, _abi.MOE_COMBINE):
        dims, symbol = moe.launch_geometry(entry, desc, max_tokens)
        if symbol:
            out.append((entry, symbol, dims.grid, dims.block))
    return out


def fp8_entry(op_kind: OperationKind, shape, family: str, max_tokens: int, paged: bool = True,
              digest: str | None = None, scale_mode: int | None = None) -> CatalogEntry:
    """The catalog entry of one operation for this build's code object and
    a profile of max_tokens rows: the manifest family of the symbol the
    launch geometry picks, the workspace the C ABI sizes (256-byte aligned),
    compute capability 9.5. family: "w8a16" or "w8a8" for the dense kinds
    (ignored for ExpertMlp); scale_mode: the weights' (per channel by
    default)."""
    from . import _abi, fp8, manifest, moe
    digest = digest or code_object_digest()
    block = scale_mode == _abi.LF_FP8_SCALE_BLOCK128
    if op_kind == OperationKind.EXPERT_MLP:
        symbol = expert_mlp_steps(shape, max_tokens)[0][1]
        workspace = moe.workspace_bytes(_descriptor(shape), max_tokens)
        capability = Capability.EXPERT_MLP
    elif op_kind == OperationKind.GATED_MLP:
        entry = (_abi.ENTRY_W8A8_GATED_MLP_B128 if block else _abi.ENTRY_W8A8_GATED_MLP) if family == "w8a8" \
            else (_abi.ENTRY_W8A16_GATED_MLP_B128 if block else _abi.ENTRY_W8A16_GATED_MLP)
        geometry = fp8.gated_mlp_geometry(shape.hidden_size, shape.intermediate_size, max_tokens, entry)
        if geometry is None:
            raise CatalogError("MissingKernel")
        symbol = geometry[1]
        workspace = _abi.lib().lunaflux_fp8_gated_mlp_workspace_bytes(entry, shape.hidden_size,
                                                                     shape.intermediate_size, max_tokens)
        capability = Capability.GATED_MLP
    elif op_kind in (OperationKind.OUTPUT_PROJECTION, OperationKind.LANGUAGE_MODEL_HEAD):
        key = (family, "dense")
        entry = fp8._BLOCK_ENTRIES[key] if block else (
            _abi.ENTRY_W8A16_DENSE if family == "w8a16" else _abi.ENTRY_W8A8_DENSE_AQ)
        n, k = shape.output_width, shape.input_width
        symbol = fp8.launch_geometry(entry, n, k, max_tokens)[1]
        workspace = (fp8.w8a16_workspace_bytes(entry, n, k, max_tokens) if family == "w8a16"
                     else fp8.w8a8_workspace_bytes(entry, n, k, max_tokens))
        capability = Capability.DENSE_PROJECTION
    else:
        raise CatalogError("MissingKernel")
    family_id = manifest.family_of(symbol)
    if family_id is None:
        raise CatalogError("MissingKernel")
    impl = ContentAddressedAot(digest, family_id)
    if paged:
        sem = ExecutionSemantics(None, (RuntimeInput.STEP_COUNTS,))
        return CatalogEntry.new_paged_v3(op_kind, shape, capability, sem, 9, 5, impl, workspace, 256)
    return CatalogEntry.new(op_kind, shape, capability, 9, 5, impl, workspace, 256)
