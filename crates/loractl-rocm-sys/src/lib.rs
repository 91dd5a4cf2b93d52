//! Rust binding of libloractl_rocm: the hand-written gfx950 (MI355X) kernels
//! of loractl's quantized frozen-base LoRA linear.
//!
//! [`ffi`] mirrors `include/loractl_rocm.h` one declaration to one
//! declaration (a CPU test of the repository checks names, arity and types).
//! The safe layer above it keeps the C ABI's contract:
//!
//! - every tensor is a device pointer owned by the caller ([`DevPtr`]);
//! - calls are stream-ordered and asynchronous on the context's stream;
//! - a failed call becomes an `anyhow` error carrying the library's message,
//!   in the style of the trainer's own errors (`diffusion_trainer.rs:385-400`);
//!   nothing falls back to another path.
//!
//! The seams it replaces, in `crates/loractl-core/src`:
//! `QuantBackend::quant_matmul_t` (`quant.rs:172-178`) and `QuantMatmulT`
//! (`quant.rs:210-263`) -> [`Context::quant_matmul_t`] /
//! [`Context::quant_matmul_t_bwd`]; `site()` with a quantized base and a
//! registered delta (`mmdit.rs:526-536`) -> [`Context::lora_fwd`] /
//! [`Context::lora_bwd`]; `quantize_linear_weight` (`quant.rs:74-82`) ->
//! [`Context::quantize_int4`].

#![allow(non_camel_case_types)]

use std::ffi::CStr;
use std::os::raw::c_void;

/// The C ABI, declaration for declaration.
pub mod ffi {
    use std::os::raw::{c_char, c_int, c_void};

    pub const LRQ_ABI_VERSION: c_int = 1;

    pub const LRQ_OK: c_int = 0;
    pub const LRQ_EINVAL: c_int = -1;
    pub const LRQ_EUNSUPPORTED: c_int = -2;
    pub const LRQ_EHIP: c_int = -3;
    pub const LRQ_ENOMEM: c_int = -4;

    pub const LRQ_FMT_INT4: i32 = 1;
    pub const LRQ_FMT_FP8: i32 = 2;
    pub const LRQ_FMT_INT8: i32 = 3;
    pub const LRQ_LAYOUT_ROWS: i32 = 0;
    pub const LRQ_LAYOUT_BLOCKED: i32 = 1;

    pub const LRQ_NOALLOC_SCRATCH_BYTES: u32 = 32 << 20;
    pub const LRQ_MAX_LORA_TOKENS: i64 = 259456;

    /// Opaque context (a device, a stream, a workspace).
    #[repr(C)]
    pub struct lrq_ctx {
        _private: [u8; 0],
    }

    /// `struct lrq_weight`: a frozen base weight, plain pointers and sizes.
    #[repr(C)]
    #[derive(Debug, Clone, Copy)]
    pub struct lrq_weight {
        pub format: i32,
        pub group: i32,
        pub n: i64,
        pub k: i64,
        pub data: *const c_void,
        pub scales: *const f32,
        pub per_channel: i32,
        pub layout: i32,
        pub bias: *const f32,
    }

    extern "C" {
        pub fn lrq_version() -> c_int;
        pub fn lrq_create(device: c_int, out: *mut *mut lrq_ctx) -> c_int;
        pub fn lrq_destroy(ctx: *mut lrq_ctx) -> c_int;
        pub fn lrq_set_stream(ctx: *mut lrq_ctx, stream: *mut c_void) -> c_int;
        pub fn lrq_sync(ctx: *mut lrq_ctx) -> c_int;
        pub fn lrq_last_error(ctx: *const lrq_ctx) -> *const c_char;
        pub fn lrq_reserve(ctx: *mut lrq_ctx, m: i64, n: i64, k: i64, r: i64) -> c_int;
        pub fn lrq_quantize_int4(
            ctx: *mut lrq_ctx,
            w: *const f32,
            n: i64,
            k: i64,
            group: i64,
            packed: *mut u8,
            scales: *mut f32,
        ) -> c_int;
        pub fn lrq_quantize_int8(
            ctx: *mut lrq_ctx,
            w: *const f32,
            n: i64,
            k: i64,
            group: i64,
            q: *mut i8,
            scales: *mut f32,
        ) -> c_int;
        pub fn lrq_quantize_fp8(
            ctx: *mut lrq_ctx,
            w: *const f32,
            n: i64,
            k: i64,
            per_channel: c_int,
            bytes: *mut u8,
            scales: *mut f32,
        ) -> c_int;
        pub fn lrq_requantize_fp8_int4(
            ctx: *mut lrq_ctx,
            bytes: *const u8,
            scale: *const f32,
            per_channel: c_int,
            n: i64,
            k: i64,
            group: i64,
            packed: *mut u8,
            scales: *mut f32,
        ) -> c_int;
        pub fn lrq_weight_blocked_size(
            format: c_int,
            n: i64,
            k: i64,
            group: i64,
            data_bytes: *mut i64,
            scale_count: *mut i64,
        ) -> c_int;
        pub fn lrq_weight_block(
            ctx: *mut lrq_ctx,
            rows: *const lrq_weight,
            data_out: *mut u8,
            scales_out: *mut f32,
        ) -> c_int;
        pub fn lrq_dequant(ctx: *mut lrq_ctx, w: *const lrq_weight, out: *mut f32) -> c_int;
        pub fn lrq_dequant_bf16(ctx: *mut lrq_ctx, w: *const lrq_weight, out: *mut u16) -> c_int;
        pub fn lrq_quant_matmul_t(
            ctx: *mut lrq_ctx,
            w: *const lrq_weight,
            x: *const u16,
            m: i64,
            y: *mut u16,
        ) -> c_int;
        pub fn lrq_quant_matmul_t_bwd(
            ctx: *mut lrq_ctx,
            w: *const lrq_weight,
            dy: *const u16,
            m: i64,
            dx: *mut u16,
        ) -> c_int;
        pub fn lrq_lora_fwd(
            ctx: *mut lrq_ctx,
            w: *const lrq_weight,
            x: *const u16,
            m: i64,
            a: *const u16,
            b: *const u16,
            r: i64,
            scaling: f32,
            y: *mut u16,
            t_out: *mut u16,
        ) -> c_int;
        pub fn lrq_lora_fwd_noalloc(
            ctx: *mut lrq_ctx,
            w: *const lrq_weight,
            x: *const u16,
            m: i64,
            a: *const u16,
            b: *const u16,
            r: i64,
            scaling: f32,
            y: *mut u16,
            t_out: *mut u16,
        ) -> c_int;
        pub fn lrq_lora_bwd(
            ctx: *mut lrq_ctx,
            w: *const lrq_weight,
            x: *const u16,
            dy: *const u16,
            m: i64,
            a: *const u16,
            b: *const u16,
            r: i64,
            scaling: f32,
            t: *const u16,
            dx: *mut u16,
            da: *mut f32,
            db: *mut f32,
        ) -> c_int;
        pub fn lrq_profile_enable(ctx: *mut lrq_ctx, on: c_int) -> c_int;
        pub fn lrq_profile_reset(ctx: *mut lrq_ctx) -> c_int;
        pub fn lrq_profile_count() -> c_int;
        pub fn lrq_profile_name(kid: c_int) -> *const c_char;
        pub fn lrq_profile_read(
            ctx: *mut lrq_ctx,
            kid: c_int,
            total_ms: *mut f64,
            launches: *mut i64,
        ) -> c_int;
        pub fn lrq_profile_relaunch(ctx: *mut lrq_ctx, kid: c_int, n: c_int) -> c_int;
        pub fn lrq_probe_stream_read(ctx: *mut lrq_ctx, data: *const c_void, bytes: i64) -> c_int;
        pub fn lrq_debug_force_wait_timeout(on: c_int) -> c_int;
        pub fn lrq_debug_gemm_path(path: c_int) -> c_int;
    }
}

/// Name of a library return code.
pub fn code_name(rc: i32) -> &'static str {
    match rc {
        ffi::LRQ_OK => "LRQ_OK",
        ffi::LRQ_EINVAL => "LRQ_EINVAL",
        ffi::LRQ_EUNSUPPORTED => "LRQ_EUNSUPPORTED",
        ffi::LRQ_EHIP => "LRQ_EHIP",
        ffi::LRQ_ENOMEM => "LRQ_ENOMEM",
        _ => "unknown",
    }
}

/// A device address owned by the caller (a HIP allocation, e.g. the buffer
/// behind a burn Rocm tensor). The binding never dereferences it on the host.
#[derive(Debug, Clone, Copy, PartialEq, Eq)]
pub struct DevPtr(pub *mut c_void);

// A device address is a number to the host: it is never dereferenced here,
// so moving or sharing it across threads is sound (autodiff keeps weight
// descriptors in backward state, which must be Send).
unsafe impl Send for DevPtr {}
unsafe impl Sync for DevPtr {}

impl DevPtr {
    pub const NULL: DevPtr = DevPtr(std::ptr::null_mut());
    fn c<T>(self) -> *const T {
        self.0 as *const T
    }
    fn m<T>(self) -> *mut T {
        self.0 as *mut T
    }
}

/// Packed format of a frozen weight.
#[derive(Debug, Clone, Copy, PartialEq, Eq)]
pub enum Format {
    /// int4 nibbles `q + 8` with one f32 scale per `group` inputs of a row.
    Int4 { group: i32 },
    /// e4m3fn bytes with one f32 scale per output row, or one for the tensor.
    Fp8 { per_channel: bool },
    /// int8 bytes `q` (two's complement) with one f32 scale per `group` inputs of a row.
    Int8 { group: i32 },
}

/// A frozen weight in device memory, file layout `[d_out = n, d_in = k]`
/// (`mmdit.rs:413-444`). `blocked` says whether `data`/`scales` hold the
/// layout the fused calls read (see [`Context::block`]).
#[derive(Debug, Clone, Copy)]
pub struct Weight {
    pub format: Format,
    pub n: i64,
    pub k: i64,
    pub data: DevPtr,
    pub scales: DevPtr,
    pub bias: DevPtr,
    pub blocked: bool,
}

impl Weight {
    pub fn desc(&self) -> ffi::lrq_weight {
        let (format, group, per_channel) = match self.format {
            Format::Int4 { group } => (ffi::LRQ_FMT_INT4, group, 0),
            Format::Fp8 { per_channel } => (ffi::LRQ_FMT_FP8, 0, per_channel as i32),
            Format::Int8 { group } => (ffi::LRQ_FMT_INT8, group, 0),
        };
        ffi::lrq_weight {
            format,
            group,
            n: self.n,
            k: self.k,
            data: self.data.c(),
            scales: self.scales.c(),
            per_channel,
            layout: if self.blocked { ffi::LRQ_LAYOUT_BLOCKED } else { ffi::LRQ_LAYOUT_ROWS },
            bias: self.bias.c(),
        }
    }

    /// Bytes of packed data and count of f32 scales of the blocked layout
    /// (both sections); fp8 scales keep their shape (count 0).
    pub fn blocked_size(&self) -> anyhow::Result<(i64, i64)> {
        let d = self.desc();
        let (mut bytes, mut scales) = (0i64, 0i64);
        let rc = unsafe {
            ffi::lrq_weight_blocked_size(d.format, d.n, d.k, d.group as i64, &mut bytes, &mut scales)
        };
        if rc != ffi::LRQ_OK {
            anyhow::bail!("lrq_weight_blocked_size failed ({}) for a [{}, {}] weight", code_name(rc), d.n, d.k);
        }
        Ok((bytes, scales))
    }
}

/// One library context: a device, the stream its calls are ordered on, and
/// the workspace of the fused calls. Owned by one thread at a time (the
/// trainer's step loop is single-threaded, `train.rs:21-27`): `Send`, not
/// `Sync`.
pub struct Context {
    raw: *mut ffi::lrq_ctx,
}

unsafe impl Send for Context {}

impl Context {
    /// A context on HIP device `device`, on the device's null stream until
    /// [`Context::set_stream`].
    pub fn new(device: i32) -> anyhow::Result<Self> {
        let mut raw = std::ptr::null_mut();
        let rc = unsafe { ffi::lrq_create(device, &mut raw) };
        if rc != ffi::LRQ_OK || raw.is_null() {
            anyhow::bail!(
                "compute.backend rocm: no context on HIP device {device} ({}): is a gfx950 GPU visible?",
                code_name(rc)
            );
        }
        Ok(Self { raw })
    }

    fn check(&self, rc: i32, what: &str) -> anyhow::Result<()> {
        if rc == ffi::LRQ_OK {
            return Ok(());
        }
        let msg = unsafe { CStr::from_ptr(ffi::lrq_last_error(self.raw)) }.to_string_lossy().into_owned();
        anyhow::bail!("{what} failed ({}): {msg}", code_name(rc))
    }

    /// Order every later call on `stream` (a `hipStream_t`; null = the null stream).
    pub fn set_stream(&mut self, stream: *mut c_void) -> anyhow::Result<()> {
        let rc = unsafe { ffi::lrq_set_stream(self.raw, stream) };
        self.check(rc, "lrq_set_stream")
    }

    pub fn sync(&self) -> anyhow::Result<()> {
        let rc = unsafe { ffi::lrq_sync(self.raw) };
        self.check(rc, "lrq_sync")
    }

    /// Size the workspace once for the largest site, so the step's calls
    /// never allocate.
    pub fn reserve(&mut self, m: i64, n: i64, k: i64, r: i64) -> anyhow::Result<()> {
        let rc = unsafe { ffi::lrq_reserve(self.raw, m, n, k, r) };
        self.check(rc, "lrq_reserve")
    }

    /// `quantize_linear_weight` at Q4S (`quant.rs:74-82`): f32 `[n, k]` ->
    /// packed `[n, k/2]` + scales `[n, k/group]`, row layout.
    pub fn quantize_int4(
        &mut self,
        w: DevPtr,
        n: i64,
        k: i64,
        group: i64,
        packed: DevPtr,
        scales: DevPtr,
    ) -> anyhow::Result<()> {
        let rc = unsafe { ffi::lrq_quantize_int4(self.raw, w.c(), n, k, group, packed.m(), scales.m()) };
        self.check(rc, "lrq_quantize_int4")
    }

    /// The same at Q8S (`quant.rs:156-162`): f32 `[n, k]` -> int8 `q [n, k]`
    /// + scales `[n, k/group]`, row layout.
    pub fn quantize_int8(
        &mut self,
        w: DevPtr,
        n: i64,
        k: i64,
        group: i64,
        q: DevPtr,
        scales: DevPtr,
    ) -> anyhow::Result<()> {
        let rc = unsafe { ffi::lrq_quantize_int8(self.raw, w.c(), n, k, group, q.m() as *mut i8, scales.m()) };
        self.check(rc, "lrq_quantize_int8")
    }

    /// An fp8 checkpoint tensor (e4m3fn bytes and its scale) re-quantized
    /// to int4 on the device (the load pass of `diffusion_trainer.rs:1143-1169`
    /// without the f32 copy).
    #[allow(clippy::too_many_arguments)]
    pub fn requantize_fp8_int4(
        &mut self,
        bytes: DevPtr,
        scale: DevPtr,
        per_channel: bool,
        n: i64,
        k: i64,
        group: i64,
        packed: DevPtr,
        scales: DevPtr,
    ) -> anyhow::Result<()> {
        let rc = unsafe {
            ffi::lrq_requantize_fp8_int4(
                self.raw,
                bytes.c(),
                scale.c(),
                per_channel as i32,
                n,
                k,
                group,
                packed.m(),
                scales.m(),
            )
        };
        self.check(rc, "lrq_requantize_fp8_int4")
    }

    /// Re-lay a row-layout weight into the blocked layout the fused calls
    /// read (buffers sized by [`Weight::blocked_size`]); once per frozen weight.
    pub fn block(&mut self, rows: &Weight, data_out: DevPtr, scales_out: DevPtr) -> anyhow::Result<Weight> {
        anyhow::ensure!(!rows.blocked, "lrq_weight_block takes a row-layout weight");
        let d = rows.desc();
        let rc = unsafe { ffi::lrq_weight_block(self.raw, &d, data_out.m(), scales_out.m()) };
        self.check(rc, "lrq_weight_block")?;
        let scales = match rows.format {
            Format::Int4 { .. } | Format::Int8 { .. } => scales_out,
            Format::Fp8 { .. } => rows.scales,
        };
        Ok(Weight { data: data_out, scales, blocked: true, ..*rows })
    }

    /// f32 `[n, k]` dequantized weight (bit-exact; the parity surface).
    pub fn dequant(&mut self, w: &Weight, out: DevPtr) -> anyhow::Result<()> {
        let d = w.desc();
        let rc = unsafe { ffi::lrq_dequant(self.raw, &d, out.m()) };
        self.check(rc, "lrq_dequant")
    }

    /// `QuantBackend::quant_matmul_t`: `y[m, n] = x[m, k] . dequant(w)^T (+bias)`, bf16.
    pub fn quant_matmul_t(&mut self, w: &Weight, x: DevPtr, m: i64, y: DevPtr) -> anyhow::Result<()> {
        let d = w.desc();
        let rc = unsafe { ffi::lrq_quant_matmul_t(self.raw, &d, x.c(), m, y.m()) };
        self.check(rc, "lrq_quant_matmul_t")
    }

    /// `QuantMatmulT::backward`: `dx[m, k] = dy[m, n] . dequant(w)`, bf16.
    pub fn quant_matmul_t_bwd(&mut self, w: &Weight, dy: DevPtr, m: i64, dx: DevPtr) -> anyhow::Result<()> {
        let d = w.desc();
        let rc = unsafe { ffi::lrq_quant_matmul_t_bwd(self.raw, &d, dy.c(), m, dx.m()) };
        self.check(rc, "lrq_quant_matmul_t_bwd")
    }

    /// The fused site forward: `y = x . dequant(w)^T (+bias) + s . (x . A) . B`
    /// with `t = s . x . A` (bf16 `[m, r]`) saved for the backward.
    #[allow(clippy::too_many_arguments)]
    pub fn lora_fwd(
        &mut self,
        w: &Weight,
        x: DevPtr,
        m: i64,
        a: DevPtr,
        b: DevPtr,
        r: i64,
        scaling: f32,
        y: DevPtr,
        t: DevPtr,
    ) -> anyhow::Result<()> {
        let d = w.desc();
        let rc = unsafe { ffi::lrq_lora_fwd(self.raw, &d, x.c(), m, a.c(), b.c(), r, scaling, y.m(), t.m()) };
        self.check(rc, "lrq_lora_fwd")
    }

    /// The fused site backward: dx (bf16), dA and dB (f32); a null output is
    /// skipped. No gradient is formed for the frozen weight.
    #[allow(clippy::too_many_arguments)]
    pub fn lora_bwd(
        &mut self,
        w: &Weight,
        x: DevPtr,
        dy: DevPtr,
        m: i64,
        a: DevPtr,
        b: DevPtr,
        r: i64,
        scaling: f32,
        t: DevPtr,
        dx: DevPtr,
        da: DevPtr,
        db: DevPtr,
    ) -> anyhow::Result<()> {
        let d = w.desc();
        let rc = unsafe {
            ffi::lrq_lora_bwd(
                self.raw,
                &d,
                x.c(),
                dy.c(),
                m,
                a.c(),
                b.c(),
                r,
                scaling,
                t.c(),
                dx.m(),
                da.m(),
                db.m(),
            )
        };
        self.check(rc, "lrq_lora_bwd")
    }
}

impl Drop for Context {
    fn drop(&mut self) {
        // waits for the context's stream, then frees its workspace
        unsafe {
            ffi::lrq_destroy(self.raw);
        }
    }
}

#[cfg(test)]
mod tests {
    use super::*;

    #[test]
    fn abi_version_matches() {
        assert_eq!(unsafe { ffi::lrq_version() }, ffi::LRQ_ABI_VERSION);
    }

    #[test]
    fn blocked_size_needs_no_gpu() {
        // int4 12288 x 3072, group 64: two sections of 192 x 48 blocks of
        // 2 KiB each
        let w = Weight {
            format: Format::Int4 { group: 64 },
            n: 12288,
            k: 3072,
            data: DevPtr::NULL,
            scales: DevPtr::NULL,
            bias: DevPtr::NULL,
            blocked: false,
        };
        let (bytes, _) = w.blocked_size().unwrap();
        assert_eq!(bytes, 2 * 192 * 48 * 2048);
    }

    #[test]
    fn null_context_is_an_error_not_a_crash() {
        assert_eq!(unsafe { ffi::lrq_sync(std::ptr::null_mut()) }, ffi::LRQ_EINVAL);
    }

    #[test]
    #[ignore = "needs a gfx950 GPU"]
    fn context_on_device_zero() {
        let ctx = Context::new(0).unwrap();
        ctx.sync().unwrap();
    }
}
