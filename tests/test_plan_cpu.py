"""The plan and catalog vocabulary with the MoE operation (lunaflux_amd/plan.py),
on the CPU: the reference's catalog rules kept (kernels/catalog/entry.mbt:
54-228, execution.mbt:136-175, catalog.mbt:143-350, the cases of its
catalog_test.mbt and paged_v3_test.mbt that apply), the ExpertMlp rows
added, and the entries this build's code object provides."""
import pytest

from lunaflux_amd import _abi, fp8, manifest, moe
from lunaflux_amd import plan as P

OK = P.OperationKind
DIGEST = "fedcba9876543210fedcba9876543210fedcba9876543210fedcba9876543210"
AOT = P.ContentAddressedAot(DIGEST, 9)
MIXTRAL = P.ExpertMlpShape(4096, 14336, 8, 2, 0, 0)
FINE = P.ExpertMlpShape(2048, 1408, 64, 6, 1, 128)
STEP = (P.RuntimeInput.STEP_COUNTS,)


def expert_op(op_id=7, shape=MIXTRAL, workspace=0, paged=True):
    return P.PlanOperation.expert_mlp(op_id, 1, 2, 10, 11, 12, 13, 3, shape, workspace, paged=paged)


def expert_entry(shape=MIXTRAL, paged=True, target=(9, 5), workspace=0, alignment=256, impl=AOT):
    if paged:
        return P.CatalogEntry.new_paged_v3(OK.EXPERT_MLP, shape, P.Capability.EXPERT_MLP,
                                           P.ExecutionSemantics(None, STEP), *target, impl, workspace, alignment)
    return P.CatalogEntry.new(OK.EXPERT_MLP, shape, P.Capability.EXPERT_MLP, *target, impl, workspace, alignment)


def invalid(rule, fn):
    with pytest.raises(P.CatalogError) as e:
        fn()
    assert (e.value.kind, e.value.rule) == ("InvalidCatalog", rule)


def test_expert_mlp_entries_are_legal_in_both_catalog_versions():
    assert expert_entry(paged=False).semantic_version == P.SEMANTIC_V1
    e = expert_entry(paged=True)
    assert e.semantic_version == P.SEMANTIC_V3 and e.execution_semantics.runtime_inputs == STEP


def test_entry_shape_and_capability_must_match_its_operation_semantics():
    # the reference's rule for every kind, with the ExpertMlp rows added
    invalid("OperationShapeMismatch", lambda: P.CatalogEntry.new(
        OK.EXPERT_MLP, P.GatedMlpShape(4096, 14336), P.Capability.EXPERT_MLP, 9, 5, AOT, 0, 256))
    invalid("OperationShapeMismatch", lambda: P.CatalogEntry.new(
        OK.GATED_MLP, MIXTRAL, P.Capability.GATED_MLP, 9, 5, AOT, 0, 256))
    invalid("OperationCapabilityMismatch", lambda: P.CatalogEntry.new(
        OK.EXPERT_MLP, MIXTRAL, P.Capability.GATED_MLP, 9, 5, AOT, 0, 256))
    invalid("OperationCapabilityMismatch", lambda: P.CatalogEntry.new(
        OK.GATED_MLP, P.GatedMlpShape(4096, 14336), P.Capability.EXPERT_MLP, 9, 5, AOT, 0, 256))
    # unchanged reference rows: dense projection capability for o and the head
    for kind in (OK.OUTPUT_PROJECTION, OK.LANGUAGE_MODEL_HEAD):
        P.CatalogEntry.new(kind, P.ProjectionShape(4096, 4096), P.Capability.DENSE_PROJECTION, 9, 5, AOT, 0, 1)
    invalid("OperationCapabilityMismatch", lambda: P.CatalogEntry.new(
        OK.QKV_PROJECTION, P.ProjectionShape(4096, 6144), P.Capability.DENSE_PROJECTION, 9, 5, AOT, 0, 1))


def test_version_alignment_and_target_validation_fail_closed():
    invalid("InvalidComputeCapability", lambda: expert_entry(target=(0, 5)))
    invalid("InvalidWorkspaceBytes", lambda: expert_entry(workspace=-1))
    invalid("InvalidWorkspaceAlignment", lambda: expert_entry(alignment=3))
    invalid("InvalidWorkspaceAlignment", lambda: expert_entry(alignment=1 << 17))
    invalid("UnsupportedSemanticVersion", lambda: P.CatalogEntry.new(
        OK.EXPERT_MLP, MIXTRAL, P.Capability.EXPERT_MLP, 9, 5, AOT, 0, 256, semantic_version=P.SEMANTIC_V3))


def test_paged_expert_mlp_is_stateless_with_step_counts_only():
    layer = 0
    for sem in (P.ExecutionSemantics(None, ()),
                P.ExecutionSemantics(None, (P.RuntimeInput.STEP_COUNTS, P.RuntimeInput.QUERY_POSITIONS)),
                P.ExecutionSemantics(layer, STEP),
                P.ExecutionSemantics(None, STEP, P.KvCacheReadWrite(layer))):
        invalid("InvalidExecutionSemantics", lambda sem=sem: P.CatalogEntry.new_paged_v3(
            OK.EXPERT_MLP, MIXTRAL, P.Capability.EXPERT_MLP, sem, 9, 5, AOT, 0, 256))


def test_vendor_gemm_is_illegal_for_expert_mlp():
    invalid("InvalidVendorImplementationKind", lambda: expert_entry(paged=False, impl=P.VendorBf16Gemm()))
    invalid("InvalidVendorImplementationKind", lambda: expert_entry(paged=True, impl=P.VendorBf16Gemm()))
    # the reference's own row: legal for a dense projection in v1, never in v3
    P.CatalogEntry.new(OK.OUTPUT_PROJECTION, P.ProjectionShape(64, 64), P.Capability.DENSE_PROJECTION, 9, 5,
                       P.VendorBf16Gemm(), 0, 1)
    invalid("InvalidWorkspaceAlignment", lambda: P.CatalogEntry.new(
        OK.OUTPUT_PROJECTION, P.ProjectionShape(64, 64), P.Capability.DENSE_PROJECTION, 9, 5,
        P.VendorBf16Gemm(), 64, 128))


@pytest.mark.parametrize("dims", [
    (4096, 14336, 8, 2, 0, 0), (2048, 1408, 64, 6, 1, 128), (128, 128, 1, 1, 0, 0), (128, 256, 256, 16, 1, 0),
    (0, 128, 8, 2, 0, 0), (4096, 14336, 257, 2, 0, 0), (4096, 14336, 8, 9, 0, 0), (4096, 14336, 32, 17, 0, 0),
    (4096, 14336, 8, 2, 2, 0), (4000, 14336, 8, 2, 0, 0), (4096, 14336, 8, 2, 0, 64),
    (8192, 1408, 64, 6, 1, 128), (2048, 1408, 64, 0, 1, 128),
])
def test_expert_mlp_shape_matches_the_routing_descriptor(dims):
    """The plan shape accepts exactly the dimensions the C ABI's routing
    descriptor does."""
    try:
        moe.moe_descriptor(dims[2], dims[3], dims[4], dims[0], dims[1], dims[5])
        c_ok = True
    except fp8.DeviceError:
        c_ok = False
    try:
        P.ExpertMlpShape(*dims)
        plan_ok = True
    except P.PlanValidationError as e:
        assert e.kind == "InvalidShape"
        plan_ok = False
    assert plan_ok == c_ok, dims


def test_expert_mlp_operation_contract():
    op = expert_op()
    assert op.kind == OK.EXPERT_MLP and op.runtime_inputs == STEP and op.kv_layer is None
    assert [type(v).__name__ for v in op.inputs] == ["Activation", "Activation"] + ["Tensor"] * 4
    assert expert_op(paged=False).runtime_inputs == ()
    with pytest.raises(P.PlanValidationError) as e:
        expert_op(workspace=-1)
    assert e.value.kind == "InvalidWorkspaceBound"
    with pytest.raises(P.PlanValidationError) as e:
        P.PlanOperation.new_stateless(1, OK.ROTARY_EMBEDDING, [P.Activation(0)], [P.Activation(1)],
                                      P.RotaryShape(4, 2, 4, 1e4), P.Capability.ROTARY_EMBEDDING, 0)
    assert (e.value.kind, e.value.detail) == ("InvalidGraph", "KvExecutionContract")
    with pytest.raises(P.PlanValidationError):
        P.PlanOperation.new_stateless(1, OK.EXPERT_MLP, [], [P.Activation(1)], MIXTRAL, P.Capability.EXPERT_MLP, 0)


def dense_gated(op_id=5):
    return P.PlanOperation.new_with_runtime_inputs(5, OK.GATED_MLP, [P.Activation(0), P.Tensor(1), P.Tensor(2),
                                                                     P.Tensor(3)], [P.Activation(4)],
                                                   P.GatedMlpShape(4096, 14336), P.Capability.GATED_MLP, 0, STEP)


def gated_entry(target=(9, 5)):
    return P.CatalogEntry.new_paged_v3(OK.GATED_MLP, P.GatedMlpShape(4096, 14336), P.Capability.GATED_MLP,
                                       P.ExecutionSemantics(None, STEP), *target, P.ContentAddressedAot(DIGEST, 11),
                                       1 << 20, 256)


def test_catalog_resolves_one_exact_binding_per_operation():
    cat = P.KernelCatalog(P.CATALOG_V3, [gated_entry(), expert_entry(workspace=1000)])
    b = cat.resolve([dense_gated(), expert_op()], P.GFX950, workspace_limit=1 << 30)
    assert [x.operation_id for x in b] == [5, 7]
    assert b[1].implementation == AOT and b[1].workspace_bytes == 1024   # rounded up to 256
    assert b[1].capability == P.Capability.EXPERT_MLP


def test_missing_ambiguous_target_and_workspace_failures():
    def fails(kind, cat, ops, limit=1 << 30):
        with pytest.raises(P.CatalogError) as e:
            cat.resolve(ops, P.GFX950, limit)
        assert e.value.kind == kind and e.value.operation == ops[-1].id
    fails("MissingKernel", P.KernelCatalog(P.CATALOG_V3, [gated_entry()]), [dense_gated(), expert_op()])
    # a shape that differs in one routing field does not match
    fails("MissingKernel", P.KernelCatalog(P.CATALOG_V3, [expert_entry(P.ExpertMlpShape(4096, 14336, 8, 2, 1, 0))]),
          [expert_op()])
    fails("IncompatibleTarget", P.KernelCatalog(P.CATALOG_V3, [expert_entry(target=(9, 4))]), [expert_op()])
    fails("AmbiguousKernel", P.KernelCatalog(P.CATALOG_V3, [expert_entry(), expert_entry()]), [expert_op()])
    fails("WorkspaceRequirementMismatch", P.KernelCatalog(P.CATALOG_V3, [expert_entry(workspace=256)]),
          [expert_op(workspace=4096)])
    fails("WorkspaceLimitExceeded", P.KernelCatalog(P.CATALOG_V3, [expert_entry(workspace=4096)]),
          [expert_op()], limit=1024)
    # a v1 (stateless) entry does not match a paged operation, nor a v3
    # entry a stateless one; catalog and entry versions do not cross
    fails("MissingKernel", P.KernelCatalog(P.CATALOG_V1, [expert_entry(paged=False)]), [expert_op()])
    fails("MissingKernel", P.KernelCatalog(P.CATALOG_V3, [expert_entry()]), [expert_op(paged=False)])
    with pytest.raises(P.CatalogError) as e:
        P.KernelCatalog(P.CATALOG_V3, [expert_entry(paged=False)])
    assert e.value.rule == "CatalogSemanticVersionMismatch"


def test_this_builds_expert_mlp_entries():
    """Entries of the code object: the MoE family, the C ABI's workspace,
    the launch steps the geometry gives each profile."""
    for shape, t, want in [
        (MIXTRAL, 1024, ["lf_moe_route", "lf_moe_sort_count", "lf_moe_sort", "lf_moe_quant_tokens",
                         "lf_moe_gate_up_t256", "lf_moe_down_t256_aq", "lf_moe_combine"]),
        (FINE, 4096, ["lf_moe_route", "lf_moe_sort_count", "lf_moe_sort", "lf_moe_quant_tokens",
                      "lf_moe_gate_up_t256_b128_q", "lf_moe_down_t256_b128", "lf_moe_combine"]),
        (FINE, 32, ["lf_moe_route_sort", "lf_moe_gate_up_gemv", "lf_moe_quant_hidden", "lf_moe_down_gemv",
                    "lf_moe_combine"]),
    ]:
        steps = P.expert_mlp_steps(shape, t)
        assert [s[1] for s in steps] == want
        assert {manifest.family_of(s[1]) for s in steps} == {9}
        e = P.fp8_entry(OK.EXPERT_MLP, shape, "w8a8", t, digest=DIGEST)
        desc = moe.moe_descriptor(shape.experts, shape.top_k, shape.route_mode, shape.hidden_size,
                                  shape.intermediate_size, shape.scale_group)
        assert e.implementation == P.ContentAddressedAot(DIGEST, 9)
        assert e.workspace_bytes == moe.workspace_bytes(desc, t) and e.workspace_alignment == 256
        b = P.KernelCatalog(P.CATALOG_V3, [e]).resolve([expert_op(shape=shape)], P.GFX950, 1 << 40)
        assert b[0].workspace_bytes >= e.workspace_bytes


def test_this_builds_dense_entries():
    gm = P.GatedMlpShape(4096, 14336)
    e = P.fp8_entry(OK.GATED_MLP, gm, "w8a8", 2048, digest=DIGEST)
    assert e.implementation.family_id == 11
    assert e.workspace_bytes == _abi.lib().lunaflux_fp8_gated_mlp_workspace_bytes(
        _abi.ENTRY_W8A8_GATED_MLP, 4096, 14336, 2048)
    assert P.fp8_entry(OK.GATED_MLP, gm, "w8a8", 2048, digest=DIGEST,
                       scale_mode=_abi.LF_FP8_SCALE_BLOCK128).implementation.family_id == 21
    assert P.fp8_entry(OK.GATED_MLP, gm, "w8a16", 32, digest=DIGEST).implementation.family_id == 10
    b = P.fp8_entry(OK.GATED_MLP, gm, "w8a16", 32, digest=DIGEST, scale_mode=_abi.LF_FP8_SCALE_BLOCK128)
    assert b.implementation.family_id == 22 and b.workspace_bytes == _abi.lib().lunaflux_fp8_gated_mlp_workspace_bytes(
        _abi.ENTRY_W8A16_GATED_MLP_B128, 4096, 14336, 32)
    o = P.ProjectionShape(4096, 4096)
    assert P.fp8_entry(OK.OUTPUT_PROJECTION, o, "w8a8", 2048, digest=DIGEST).implementation.family_id == 12
    assert P.fp8_entry(OK.OUTPUT_PROJECTION, o, "w8a16", 32, digest=DIGEST).implementation.family_id == 3
    assert P.fp8_entry(OK.OUTPUT_PROJECTION, o, "w8a16", 32, digest=DIGEST,
                       scale_mode=_abi.LF_FP8_SCALE_BLOCK128).implementation.family_id == 15
    e = P.fp8_entry(OK.LANGUAGE_MODEL_HEAD, P.ProjectionShape(4096, 128256), "w8a16", 32, digest=DIGEST, paged=False)
    assert e.semantic_version == P.SEMANTIC_V1 and e.implementation.family_id == 3
