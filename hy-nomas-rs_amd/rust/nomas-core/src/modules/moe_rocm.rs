//! MI355X (gfx950) drop-in for the MoE feed-forward block and the SwiGLU
//! feed-forward of nomas-core, over `nomas-moe-sys` (libnomas_moe.so).
//!
//! This file goes to `nomas-core/src/modules/moe_rocm.rs`; with the `rocm`
//! feature, `modules/mod.rs` declares it and `modules/block.rs` imports its
//! `MoeLayer` instead of the candle one, and builds `SwiGluRocm` for dense
//! SwiGLU blocks (three small edits, listed in INTEGRATION.md).  The
//! candle `MoeLayer` in moe.rs stays as it is.  The public surface is the
//! reference's:
//! `MoeLayer::from_source(&Weights, path, dim, hidden, &MoeConfig)`,
//! `forward(&Tensor) -> Result<Tensor>`, `n_params()` (moe.rs:26-114), so
//! `BlockFfn::Moe(Box<MoeLayer>)` and its caller (block.rs:14-19,97-100) do not
//! change.
//!
//! Parameters are materialised by the reference's own code: every `Lin` is
//! built with `Lin::from_source` exactly as moe.rs:33-54 and mlp.rs:30-34 do
//! (so `Weights::Loaded` reads `{path}.router.weight`,
//! `{path}.experts.{e}.{gate,up,down}.{weight,bias}` through `vb.get` with the
//! reference's shapes and errors, mod.rs:69-77, and `Weights::Random` draws the
//! reference's xavier streams, mod.rs:80-95), then their bytes go to
//! `nomas_moe_from_host`, which packs them for the GEMMs and keeps them on the
//! GPU.  `forward` takes candle CPU tensors (the reference's device): the rows
//! are copied to the GPU, the forward runs there, the result comes back.
use std::ffi::CStr;
use std::os::raw::{c_int, c_void};
use std::sync::Mutex;

use candle_core::{CpuStorage, DType, Device, Result, Storage, Tensor};
use nomas_moe_sys as sys;

use super::{Lin, Weights};
use crate::config::MoeConfig;

/// HIP device the handles live on.
const HIP_DEVICE: c_int = 0;

fn err(msg: String) -> candle_core::Error {
    candle_core::Error::Msg(msg)
}

/// The library's dtype code; anything but F32, BF16 and F16 is an error (the
/// reference's models are one of these, config.rs:30-39).
fn dtype_code(d: DType) -> Result<c_int> {
    match d {
        DType::F32 => Ok(sys::NOMAS_F32),
        DType::BF16 => Ok(sys::NOMAS_BF16),
        DType::F16 => Ok(sys::NOMAS_F16),
        other => Err(err(format!(
            "the MI355X feed-forward supports F32, BF16 and F16 models, not {other:?}"
        ))),
    }
}

/// A library status as a candle error carrying the library's message
/// (lifted to `nomas_core::Error::Candle` by `?` at the block, as the
/// reference's own errors are).
fn check(rc: c_int) -> Result<()> {
    if rc == sys::NOMAS_OK {
        return Ok(());
    }
    let msg = unsafe { CStr::from_ptr(sys::nomas_moe_last_error()) }.to_string_lossy().into_owned();
    Err(err(msg))
}

/// Row-major bytes of a CPU tensor in its own dtype (little-endian, as the C
/// ABI takes them).
fn host_bytes(t: &Tensor) -> Result<Vec<u8>> {
    let t = t.contiguous()?;
    let n = t.elem_count() * t.dtype().size_in_bytes();
    let (st, layout) = t.storage_and_layout();
    let off = layout.start_offset();
    let p: *const u8 = match &*st {
        Storage::Cpu(CpuStorage::F32(v)) => v[off..].as_ptr().cast(),
        Storage::Cpu(CpuStorage::BF16(v)) => v[off..].as_ptr().cast(),
        Storage::Cpu(CpuStorage::F16(v)) => v[off..].as_ptr().cast(),
        Storage::Cpu(_) => {
            dtype_code(t.dtype())?;
            unreachable!()
        }
        _ => return Err(err("the MI355X feed-forward takes candle CPU tensors".into())),
    };
    Ok(unsafe { std::slice::from_raw_parts(p, n) }.to_vec())
}

/// The per-expert tensors one after another: (E, ...) in the C ABI's layout.
fn stacked<'a>(ts: impl Iterator<Item = &'a Tensor>) -> Result<Vec<u8>> {
    let mut out = Vec::new();
    for t in ts {
        out.extend_from_slice(&host_bytes(t)?);
    }
    Ok(out)
}

fn bias(l: &Lin) -> &Tensor {
    // every Lin of a SwiGLU is built with bias = true (mlp.rs:30-34)
    l.bias.as_ref().expect("SwiGLU Lins carry a bias")
}

fn ptr(v: &[u8]) -> *const c_void {
    v.as_ptr().cast()
}

/// `x` -> `y` on the host through one of the library's host forwards.
fn forward_host(
    x: &Tensor,
    dtype: DType,
    dim: usize,
    f: impl FnOnce(*const c_void, *mut c_void, i64) -> c_int,
) -> Result<Tensor> {
    // Lin::fwd's matmul would reject another dtype (mod.rs:127-141)
    if x.dtype() != dtype {
        return Err(err(format!("expected a {dtype:?} input, got {:?}", x.dtype())));
    }
    let dims = x.dims().to_vec();
    if dims.last().copied() != Some(dim) {
        return Err(err(format!("expected last dim {dim}, got shape {dims:?}")));
    }
    let xb = host_bytes(x)?;
    let rows = x.elem_count() / dim; // leading dims folded as Lin::fwd does (mod.rs:132-134)
    let mut yb = vec![0u8; xb.len()];
    check(f(ptr(&xb), yb.as_mut_ptr().cast(), rows as i64))?;
    Tensor::from_raw_buffer(&yb, dtype, &dims, &Device::Cpu)
}

struct MoeHandle(*mut sys::nomas_moe_t);
// The handle may move between threads; the Mutex below keeps calls on it
// one at a time, which is what the library requires of a handle.
unsafe impl Send for MoeHandle {}

/// Router + expert bank (moe.rs:16-22) on one MI355X.
pub struct MoeLayer {
    h: Mutex<MoeHandle>,
    dtype: DType,
    dim: usize,
}

impl MoeLayer {
    /// Build from a source (moe.rs:26-62).
    pub fn from_source(
        src: &Weights<'_>,
        path: &str,
        dim: usize,
        hidden: usize,
        cfg: &MoeConfig,
    ) -> Result<Self> {
        let router = Lin::from_source(src, &format!("{path}.router"), dim, cfg.experts, false)?;
        let (mut gate, mut up, mut down) = (Vec::new(), Vec::new(), Vec::new());
        for e in 0..cfg.experts {
            let p = format!("{path}.experts.{e}");
            gate.push(Lin::from_source(src, &format!("{p}.gate"), dim, hidden, true)?);
            up.push(Lin::from_source(src, &format!("{p}.up"), dim, hidden, true)?);
            down.push(Lin::from_source(src, &format!("{p}.down"), hidden, dim, true)?);
        }
        let dense = if cfg.shared_dense > 0.0 {
            let p = format!("{path}.dense");
            Some([
                Lin::from_source(src, &format!("{p}.gate"), dim, hidden, true)?,
                Lin::from_source(src, &format!("{p}.up"), dim, hidden, true)?,
                Lin::from_source(src, &format!("{p}.down"), hidden, dim, true)?,
            ])
        } else {
            None
        };
        let dtype = router.weight.dtype();
        let code = dtype_code(dtype)?;
        let rw = host_bytes(&router.weight)?;
        let gw = stacked(gate.iter().map(|l| &l.weight))?;
        let gb = stacked(gate.iter().map(bias))?;
        let uw = stacked(up.iter().map(|l| &l.weight))?;
        let ub = stacked(up.iter().map(bias))?;
        let dw = stacked(down.iter().map(|l| &l.weight))?;
        let db = stacked(down.iter().map(bias))?;
        let dn: Option<Vec<Vec<u8>>> = match &dense {
            Some([g, u, d]) => Some(vec![
                host_bytes(&g.weight)?, host_bytes(bias(g))?,
                host_bytes(&u.weight)?, host_bytes(bias(u))?,
                host_bytes(&d.weight)?, host_bytes(bias(d))?,
            ]),
            None => None,
        };
        let dp = |i: usize| dn.as_ref().map_or(std::ptr::null(), |v| ptr(&v[i]));
        let c = sys::nomas_moe_config {
            experts: cfg.experts as i64,
            top_k: cfg.top_k as i64,
            shared_dense: cfg.shared_dense,
            seed: cfg.seed,
        };
        let mut h = std::ptr::null_mut();
        check(unsafe {
            sys::nomas_moe_from_host(
                &c, dim as i64, hidden as i64, code, HIP_DEVICE, ptr(&rw),
                ptr(&gw), ptr(&gb), ptr(&uw), ptr(&ub), ptr(&dw), ptr(&db),
                dp(0), dp(1), dp(2), dp(3), dp(4), dp(5), &mut h,
            )
        })?;
        Ok(Self { h: Mutex::new(MoeHandle(h)), dtype, dim })
    }

    /// Forward with top-k routing (moe.rs:65-109): `x` of shape `(..., D)`.
    pub fn forward(&self, x: &Tensor) -> Result<Tensor> {
        let h = self.h.lock().map_err(|_| err("MoE handle poisoned".into()))?;
        forward_host(x, self.dtype, self.dim, |xp, yp, rows| unsafe {
            sys::nomas_moe_forward_host(h.0, xp, yp, rows)
        })
    }

    /// Parameter count: router + experts, the dense branch excluded (moe.rs:112-114).
    pub fn n_params(&self) -> usize {
        let h = self.h.lock().expect("MoE handle poisoned");
        unsafe { sys::nomas_moe_n_params(h.0) as usize }
    }
}

impl Drop for MoeLayer {
    fn drop(&mut self) {
        if let Ok(h) = self.h.get_mut() {
            unsafe { sys::nomas_moe_destroy(h.0) }
        }
    }
}

struct FfnHandle(*mut sys::nomas_ffn_t);
unsafe impl Send for FfnHandle {}

/// `FeedForward::SwiGlu` (mlp.rs:13-14,39-46) on one MI355X; `FeedForward`'s
/// SwiGlu arm holds one of these with the `rocm` feature.
pub struct SwiGluRocm {
    h: Mutex<FfnHandle>,
    dtype: DType,
    dim: usize,
}

impl SwiGluRocm {
    /// `{path}.gate`, `{path}.up`, `{path}.down` as mlp.rs:30-34 builds them.
    pub fn from_source(src: &Weights<'_>, path: &str, dim: usize, hidden: usize) -> Result<Self> {
        let gate = Lin::from_source(src, &format!("{path}.gate"), dim, hidden, true)?;
        let up = Lin::from_source(src, &format!("{path}.up"), dim, hidden, true)?;
        let down = Lin::from_source(src, &format!("{path}.down"), hidden, dim, true)?;
        let dtype = gate.weight.dtype();
        let code = dtype_code(dtype)?;
        let b: Vec<Vec<u8>> = vec![
            host_bytes(&gate.weight)?, host_bytes(bias(&gate))?,
            host_bytes(&up.weight)?, host_bytes(bias(&up))?,
            host_bytes(&down.weight)?, host_bytes(bias(&down))?,
        ];
        let mut h = std::ptr::null_mut();
        check(unsafe {
            sys::nomas_ffn_from_host(
                dim as i64, hidden as i64, code, HIP_DEVICE, ptr(&b[0]), ptr(&b[1]),
                ptr(&b[2]), ptr(&b[3]), ptr(&b[4]), ptr(&b[5]), &mut h,
            )
        })?;
        Ok(Self { h: Mutex::new(FfnHandle(h)), dtype, dim })
    }

    /// `down(silu(gate(x)) * up(x))` (mlp.rs:42-46).
    pub fn forward(&self, x: &Tensor) -> Result<Tensor> {
        let h = self.h.lock().map_err(|_| err("FFN handle poisoned".into()))?;
        forward_host(x, self.dtype, self.dim, |xp, yp, rows| unsafe {
            sys::nomas_ffn_forward_host(h.0, xp, yp, rows)
        })
    }

    /// mlp.rs:50-58.
    pub fn n_params(&self) -> usize {
        let h = self.h.lock().expect("FFN handle poisoned");
        unsafe { sys::nomas_ffn_n_params(h.0) as usize }
    }
}

impl Drop for SwiGluRocm {
    fn drop(&mut self) {
        if let Ok(h) = self.h.get_mut() {
            unsafe { sys::nomas_ffn_destroy(h.0) }
        }
    }
}

#[cfg(test)]
mod tests {
    //! The reference's own MoE tests (moe.rs:123-150) against the drop-in,
    //! plus equality with the candle MoeLayer on the same random weights.
    use super::*;

    fn cfg() -> MoeConfig {
        MoeConfig { experts: 4, top_k: 2, shared_dense: 0.0, seed: 1 }
    }

    #[test]
    fn moe_output_shape_and_finiteness() {
        let dev = Device::Cpu;
        let moe = MoeLayer::from_source(&Weights::random(4, DType::F32, &dev), "blocks.0.moe", 32,
                                        64, &cfg())
            .unwrap();
        let x = crate::tensor_utils::deterministic_randn([1, 5, 32], 3, &dev).unwrap();
        let y = moe.forward(&x).unwrap();
        assert_eq!(y.dims(), vec![1, 5, 32]);
        assert!(y.flatten_all().unwrap().to_vec1::<f32>().unwrap().iter().all(|v| v.is_finite()));
    }

    #[test]
    fn matches_the_candle_moe_layer() {
        let dev = Device::Cpu;
        let src = Weights::random(4, DType::F32, &dev);
        let gpu = MoeLayer::from_source(&src, "blocks.0.moe", 256, 256, &cfg()).unwrap();
        let cpu = crate::modules::moe::MoeLayer::from_source(&src, "blocks.0.moe", 256, 256, &cfg())
            .unwrap();
        assert_eq!(gpu.n_params(), cpu.n_params());
        let x = crate::tensor_utils::deterministic_randn([2, 40, 256], 5, &dev).unwrap();
        let a = gpu.forward(&x).unwrap().flatten_all().unwrap().to_vec1::<f32>().unwrap();
        let b = cpu.forward(&x).unwrap().flatten_all().unwrap().to_vec1::<f32>().unwrap();
        let scale = b.iter().fold(0f32, |m, v| m.max(v.abs()));
        let diff = a.iter().zip(&b).fold(0f32, |m, (p, q)| m.max((p - q).abs()));
        assert!(diff <= 1e-4 * scale, "max |diff| {diff} vs max |ref| {scale}");
    }

    #[test]
    fn other_dtypes_are_an_error() {
        assert!(dtype_code(DType::F64).is_err());
        assert!(dtype_code(DType::U8).is_err());
    }
}
