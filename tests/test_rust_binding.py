"""The Rust FFI crate (crates/loractl-rocm-sys) declares exactly the C ABI of
include/loractl_rocm.h: the same functions, in number of arguments and in
each argument's and the result's type, the same struct layout and the same
constants. (CPU only; cargo is not needed to read the sources.)"""

import os
import re

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "loractl_rocm.h")
CRATE = os.path.join(ROOT, "crates", "loractl-rocm-sys")
LIB_RS = os.path.join(CRATE, "src", "lib.rs")
PATCH = os.path.join(CRATE, "patches", "0001-compute-backend-rocm.patch")

# C type -> the Rust type the binding must use for it
C2RUST = {
    "int": "c_int",
    "int32_t": "i32",
    "int64_t": "i64",
    "float": "f32",
    "double": "f64",
    "void": "()",
    "void*": "*mut c_void",
    "const void*": "*const c_void",
    "float*": "*mut f32",
    "const float*": "*const f32",
    "double*": "*mut f64",
    "int64_t*": "*mut i64",
    "int8_t*": "*mut i8",
    "uint8_t*": "*mut u8",
    "const uint8_t*": "*const u8",
    "uint16_t*": "*mut u16",
    "const uint16_t*": "*const u16",
    "const char*": "*const c_char",
    "lrq_ctx*": "*mut lrq_ctx",
    "const lrq_ctx*": "*const lrq_ctx",
    "lrq_ctx**": "*mut *mut lrq_ctx",
    "const lrq_weight*": "*const lrq_weight",
}


def _norm_c(t: str) -> str:
    t = re.sub(r"\s+", " ", t.strip())
    return re.sub(r"\s*\*", "*", t)


def _c_decls():
    txt = open(HEADER).read()
    txt = re.sub(r"/\*.*?\*/", "", txt, flags=re.S)
    txt = re.sub(r"^\s*#.*$", "", txt, flags=re.M)
    out = {}
    for m in re.finditer(r"([A-Za-z_][\w\s\*]*?)\b(lrq_[a-z0-9_]+)\s*\(([^)]*)\)\s*;", txt):
        ret, name, params = m.group(1), m.group(2), m.group(3).strip()
        args = []
        if params and params != "void":
            for p in params.split(","):
                p = p.strip()
                pm = re.match(r"(.*?)([A-Za-z_]\w*)$", p)
                args.append(_norm_c(pm.group(1)))
        out[name] = (_norm_c(ret), args)
    return out


def _rust_externs():
    txt = open(LIB_RS).read()
    block = re.search(r'extern "C" \{(.*?)\n    \}', txt, flags=re.S).group(1)
    out = {}
    for m in re.finditer(r"pub fn (lrq_[a-z0-9_]+)\s*\((.*?)\)\s*(?:->\s*([^;]+))?;", block, flags=re.S):
        name, params, ret = m.group(1), m.group(2), (m.group(3) or "()").strip()
        args = []
        for p in params.split(","):
            p = p.strip()
            if p:
                args.append(re.sub(r"\s+", " ", p.split(":", 1)[1].strip()))
        out[name] = (ret, args)
    return out


def test_every_header_function_has_an_identical_rust_extern():
    c, rust = _c_decls(), _rust_externs()
    assert len(c) >= 24
    assert set(c) == set(rust), f"only in C: {set(c) - set(rust)}; only in Rust: {set(rust) - set(c)}"
    for name, (cret, cargs) in c.items():
        rret, rargs = rust[name]
        assert C2RUST[cret] == rret, f"{name}: C returns {cret}, Rust {rret}"
        assert len(cargs) == len(rargs), f"{name}: {len(cargs)} C arguments, {len(rargs)} in Rust"
        for i, (ca, ra) in enumerate(zip(cargs, rargs)):
            assert C2RUST[ca] == ra, f"{name} argument {i}: C {ca} -> {C2RUST[ca]}, Rust {ra}"


def test_struct_layout_matches():
    h = re.sub(r"/\*.*?\*/", "", open(HEADER).read(), flags=re.S)
    body = re.search(r"typedef struct lrq_weight \{(.*?)\} lrq_weight;", h, flags=re.S).group(1)
    cfields = [(_norm_c(m.group(1)), m.group(2)) for m in re.finditer(r"([\w\s\*]+?)\s*\b(\w+);", body)]
    rs = open(LIB_RS).read()
    rbody = re.search(r"pub struct lrq_weight \{(.*?)\}", rs, flags=re.S).group(1)
    rfields = [(m.group(1), m.group(2).strip()) for m in re.finditer(r"pub (\w+): ([^,]+),", rbody)]
    assert [n for _, n in cfields] == [n for n, _ in rfields]
    for (ct, n), (_, rt) in zip(cfields, rfields):
        assert C2RUST[ct] == rt, f"field {n}: C {ct}, Rust {rt}"
    assert "#[repr(C)]\n    #[derive(Debug, Clone, Copy)]\n    pub struct lrq_weight" in rs


def test_constants_match():
    h = open(HEADER).read()
    rs = open(LIB_RS).read()
    cvals = {m.group(1): int(m.group(2)) for m in re.finditer(r"\b(LRQ_[A-Z0-9_]+)\s*=\s*(-?\d+)", h)}
    cvals["LRQ_ABI_VERSION"] = int(re.search(r"#define LRQ_ABI_VERSION (\d+)", h).group(1))
    m = re.search(r"#define LRQ_NOALLOC_SCRATCH_BYTES \((\d+)u << (\d+)\)", h)
    cvals["LRQ_NOALLOC_SCRATCH_BYTES"] = int(m.group(1)) << int(m.group(2))
    cvals["LRQ_MAX_LORA_TOKENS"] = int(re.search(r"#define LRQ_MAX_LORA_TOKENS (\d+)", h).group(1))
    for name, v in cvals.items():
        rm = re.search(rf"pub const {name}: \w+ = (-?\d+)(?: << (\d+))?;", rs)
        assert rm, f"{name} missing from the Rust binding"
        rv = int(rm.group(1)) << int(rm.group(2) or 0)
        assert rv == v, f"{name}: C {v}, Rust {rv}"


def test_build_script_compiles_every_library_source():
    src = open(os.path.join(CRATE, "build.rs")).read()
    listed = set(re.findall(r'"(lrq_\w+\.hip)"', src))
    from loractl_amd import _build
    assert listed == set(_build.SOURCES)
    assert "--offload-arch=gfx950" in src and "-packed-fp32-ops" in src
    assert 'links = "loractl_rocm"' in open(os.path.join(CRATE, "Cargo.toml")).read()


def test_patch_wires_the_backend_at_the_reference_seams():
    """The patch adds BackendKind::Rocm (config.rs), the quant and precision
    guards and the dispatch arm (diffusion_trainer.rs), the fused arm of
    site() (mmdit.rs) and the rocm feature, and every hunk names a file of
    the reference crate."""
    p = open(PATCH).read()
    files = set(re.findall(r"^\+\+\+ b/(\S+)", p, flags=re.M))
    assert files == {
        "crates/loractl-core/Cargo.toml",
        "crates/loractl-core/src/config.rs",
        "crates/loractl-core/src/diffusion_trainer.rs",
        "crates/loractl-core/src/lib.rs",
        "crates/loractl-core/src/mmdit.rs",
        "crates/loractl-core/src/quant.rs",
        "crates/loractl-core/src/rocm.rs",
    }
    added = _added(p)
    for needle in ("    Rocm,", '"rocm" | "hip" => Ok(Self::Rocm)', "BackendKind::Ndarray | BackendKind::Cuda | BackendKind::Rocm",
                   "(BackendKind::Rocm, p) if p != Precision::F32", "dispatch_checkpointing::<Rocm>(",
                   "B::fused_quant_site(x.clone(), q, Some(delta))", "B::fused_quant_site(x.clone(), q, None)",
                   'rocm = ["burn/rocm", "dep:loractl-rocm-sys"]', "fn fused_quant_site",
                   "impl QuantBackend for burn::backend::Rocm", "impl<B: Backend> Backward<B, 3> for FusedLoraSite",
                   "impl<B: Backend> Backward<B, 1> for QuantSite"):
        assert needle in added, needle
    # the rocm module calls the binding, and only through functions it declares
    rust = _rust_externs()
    for call in re.findall(r"ctx\.(\w+)\(", added):
        assert f"lrq_{call}" in rust or call in ("block",), call


def _added(p, path=None):
    """The added lines of the patch, of one file if `path` is given."""
    if path is not None:
        p = p[p.index(f"+++ b/{path}"):]
        end = p.find("\ndiff ", 1)
        p = p if end < 0 else p[:end]
    return "\n".join(l[1:] for l in p.splitlines() if l.startswith("+") and not l.startswith("+++"))


def _removed(p):
    return "\n".join(l[1:] for l in p.splitlines() if l.startswith("-") and not l.startswith("---"))


def test_patch_keeps_the_adapters_f32():
    """The reference trains the adapters (and their AdamW moments) in f32
    whenever the base is quantized (diffusion_trainer.rs:395-401). The patch
    keeps that guard, runs the model on Rocm's default f32 element, rounds
    only the site's operands to bf16, and registers the kernels' f32 dA and
    dB without a cast."""
    p = open(PATCH).read()
    assert "if config.compute.precision != Precision::F32 {" not in _removed(p)
    added = _added(p)
    assert "burn::tensor::bf16" not in _added(p, "crates/loractl-core/src/diffusion_trainer.rs")
    assert "Precision::Bf16" not in added
    rocm = _added(p, "crates/loractl-core/src/rocm.rs")
    # operands rounded at the site: x, A and B (and dy in the backward)
    assert "cast::<B>(xp, FloatDType::BF16)" in rocm and "cast::<B>(xp.primitive.clone(), FloatDType::BF16)" in rocm
    assert "(cast::<B>(a, FloatDType::BF16), cast::<B>(b, FloatDType::BF16)" in rocm
    assert rocm.count("cast::<B>(grads.consume::<B>(&ops.node), FloatDType::BF16)") == 2
    # the kernels write f32 dA [k, r] and dB [r, n]; both are registered as they are
    assert "Shape::new([k, st.r as usize]), &device, FloatDType::F32" in rocm
    assert "Shape::new([st.r as usize, n]), &device, FloatDType::F32" in rocm
    bwd = rocm[rocm.index("if let (Some(node), Some(g)) = (px, dx)"):]
    bwd = bwd[:bwd.index("\n    }\n}")]
    assert "grads.register::<B>(node.id, cast::<B>(g, FloatDType::F32));" in bwd      # dx widened to f32
    assert bwd.count("grads.register::<B>(node.id, g);") == 2                         # dA, dB as they are
    assert "FloatDType::BF16" not in bwd
    # y and dx come back widened to the model's f32
    assert rocm.count("cast::<B>(y, FloatDType::F32)") == 3


def test_patch_keeps_one_copy_of_each_quantized_weight():
    """At load, a site the library packs keeps only the library's blocked
    copy: the load pass stores the placeholder register_quant_site returns
    and skips burn's own quantization of the same values; every forward of
    a quantized site (with or without a delta) goes through the library."""
    p = open(PATCH).read()
    trainer = p[p.index("+++ b/crates/loractl-core/src/diffusion_trainer.rs"):]
    hunk = trainer[trainer.index("register_quant_site"):]
    hunk = hunk[:hunk.index("\n@@") if "\n@@" in hunk else len(hunk)]
    reg, quant = hunk.index("register_quant_site"), hunk.index("quantize_linear_weight_chunked")
    between = hunk[:quant]
    assert "q.weight = vec![placeholder];" in between and "continue;" in between and reg < quant
    assert "Err(data) => data," in between
    # no second registration after burn's chunks are built
    assert _added(p).count("crate::rocm::register_quant_site") == 1
    rocm = _added(p, "crates/loractl-core/src/rocm.rs")
    assert "-> Result<Param<Tensor<B, 2>>, TensorData>" in rocm
    assert "Param::from_tensor(Tensor::<B, 2>::zeros([1, 1], device))" in rocm
    # the base-only forward (BaseLinear::forward's quant arm) routes to the library too
    mm = _added(p, "crates/loractl-core/src/mmdit.rs")
    assert "B::fused_quant_site(x.clone(), q, None)" in mm
    assert "ctx.quant_matmul_t(" in rocm and "ctx.quant_matmul_t_bwd(" in rocm
