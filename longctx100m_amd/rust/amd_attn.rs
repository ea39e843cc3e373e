// src/amd_attn.rs of rust/longctx100m-model (add `pub mod amd_attn;` to lib.rs):
// the MI355X backend of ring_attention.rs.  The FFI mirrors
// include/longctx100m_attn.h; the two public functions keep the names, arguments
// and error texts of ring_attention.rs:139-233 and :281-475, so callers switch by
// changing the module path, and CausalAttention replaces the dense candle block
// of model.rs:223-252 as a CustomOp3 whose bwd reaches the GPU backward from
// loss.backward() (train.rs:130).  Written against candle-core 0.8.4 and half
// (both already dependencies of the crate); not compiled here (no cargo in this
// image).  tests/test_rust_binding.py checks the FFI declarations against the
// header, and tests/c/abi_ring.c (mode customop3) runs this file's exact call
// sequence from C against the oracle.
//! MI355X backend of the ring attention (liblongctx100m_attn, hand-written gfx950 kernels).
use std::ffi::{c_char, c_void, CStr};
use std::sync::Mutex;

use candle_core::{CpuStorage, CustomOp3, DType, Device, Layout, Result, Shape, Tensor};
use half::bf16;

const LC_DTYPE_F32: i32 = 0;
const LC_DTYPE_BF16: i32 = 1;

#[repr(C)]
struct LcRingDesc {
    world: i32, rank: i32, batch: i32, local_tokens: i32, heads_q: i32, heads_kv: i32,
    head_dim: i32, dtype: i32, flags: u32, causal: i32, block_q: i32, block_k: i32,
    valid_length: i64,     // -1 = None
    q_position_start: i64, // -1 = None
}

extern "C" {
    fn lc_ring_fwd_with_stats_host(d: *const LcRingDesc, qs: *const *const c_void,
        ks: *const *const c_void, vs: *const *const c_void, out: *mut c_void,
        m: *mut f32, l: *mut f32) -> i32;
    fn lc_ring_bwd_host(d: *const LcRingDesc, qs: *const *const c_void,
        ks: *const *const c_void, vs: *const *const c_void, outs: *const *const c_void,
        ms: *const *const f32, ls: *const *const f32, grad_outs: *const *const c_void,
        dq: *mut c_void, dk: *mut c_void, dv: *mut c_void) -> i32;
    fn lc_last_error() -> *const c_char;
}

fn check(rc: i32) -> Result<()> {
    if rc == 0 {
        return Ok(());
    }
    let msg = unsafe { CStr::from_ptr(lc_last_error()) }.to_string_lossy().into_owned();
    candle_core::bail!("{msg}") // the library returns ring_attention.rs:148-171's texts
}

/// A contiguous host copy of a tensor in its own dtype (f32 or bf16).
enum Host {
    F32(Vec<f32>),
    Bf16(Vec<bf16>),
}

impl Host {
    fn of(t: &Tensor) -> Result<Host> {
        let flat = t.flatten_all()?;
        match t.dtype() {
            DType::F32 => Ok(Host::F32(flat.to_vec1::<f32>()?)),
            DType::BF16 => Ok(Host::Bf16(flat.to_vec1::<bf16>()?)),
            dt => candle_core::bail!("unsupported dtype {dt:?}"),
        }
    }
    fn zeros(dtype: DType, n: usize) -> Result<Host> {
        match dtype {
            DType::F32 => Ok(Host::F32(vec![0f32; n])),
            DType::BF16 => Ok(Host::Bf16(vec![bf16::ZERO; n])),
            dt => candle_core::bail!("unsupported dtype {dt:?}"),
        }
    }
    fn ptr(&self) -> *const c_void {
        match self {
            Host::F32(v) => v.as_ptr() as *const c_void,
            Host::Bf16(v) => v.as_ptr() as *const c_void,
        }
    }
    fn mut_ptr(&mut self) -> *mut c_void {
        match self {
            Host::F32(v) => v.as_mut_ptr() as *mut c_void,
            Host::Bf16(v) => v.as_mut_ptr() as *mut c_void,
        }
    }
    fn tensor(self, shape: (usize, usize, usize, usize)) -> Result<Tensor> {
        match self {
            Host::F32(v) => Tensor::from_vec(v, shape, &Device::Cpu),
            Host::Bf16(v) => Tensor::from_vec(v, shape, &Device::Cpu),
        }
    }
    fn storage(self) -> CpuStorage {
        match self {
            Host::F32(v) => CpuStorage::F32(v),
            Host::Bf16(v) => CpuStorage::BF16(v),
        }
    }
}

fn lc_dtype(dt: DType) -> Result<i32> {
    match dt {
        DType::F32 => Ok(LC_DTYPE_F32),
        DType::BF16 => Ok(LC_DTYPE_BF16),
        dt => candle_core::bail!("unsupported dtype {dt:?}"),
    }
}

#[allow(clippy::too_many_arguments)]
fn desc(world: usize, rank: usize, (b, n, hq, d): (usize, usize, usize, usize), hkv: usize,
        dtype: DType, causal: bool, block_q: usize, block_k: usize,
        valid_length: Option<usize>, q_position_start: Option<usize>) -> Result<LcRingDesc> {
    Ok(LcRingDesc {
        world: world as i32, rank: rank as i32, batch: b as i32, local_tokens: n as i32,
        heads_q: hq as i32, heads_kv: hkv as i32, head_dim: d as i32, dtype: lc_dtype(dtype)?,
        flags: 0, causal: causal as i32, block_q: block_q as i32, block_k: block_k as i32,
        valid_length: valid_length.map_or(-1, |x| x as i64),
        q_position_start: q_position_start.map_or(-1, |x| x as i64),
    })
}

fn shard_dims(shards: &[(Tensor, Tensor, Tensor)], rank: usize)
    -> Result<((usize, usize, usize, usize), usize)> {
    let world = shards.len();
    if rank >= world {
        candle_core::bail!("rank {rank} out of range for world_size {world}");
    }
    let (q, k, _) = &shards[rank];
    if q.rank() != 4 || k.rank() != 4 {
        candle_core::bail!("q, k, v must have shape [batch, tokens, heads, head_dim]");
    }
    Ok((q.dims4()?, k.dims4()?.2))
}

/// ring_causal_attention_forward_with_stats (ring_attention.rs:139-233) on the GPU.
/// K/V may carry fewer heads than Q (native GQA); m and l come back as [B, H, n, 1] f32.
pub fn ring_causal_attention_forward_with_stats(
    shards: &[(Tensor, Tensor, Tensor)], rank: usize, causal: bool, block_q: usize,
    block_k: usize, valid_length: Option<usize>, q_position_start: Option<usize>,
) -> Result<(Tensor, Tensor, Tensor)> {
    let (dims, hkv) = shard_dims(shards, rank)?;
    let (b, n, hq, d) = dims;
    let dtype = shards[rank].0.dtype();
    let dsc = desc(shards.len(), rank, dims, hkv, dtype, causal, block_q, block_k, valid_length,
                   q_position_start)?;
    let qs = shards.iter().map(|s| Host::of(&s.0)).collect::<Result<Vec<_>>>()?;
    let ks = shards.iter().map(|s| Host::of(&s.1)).collect::<Result<Vec<_>>>()?;
    let vs = shards.iter().map(|s| Host::of(&s.2)).collect::<Result<Vec<_>>>()?;
    let (qp, kp, vp): (Vec<_>, Vec<_>, Vec<_>) = (
        qs.iter().map(Host::ptr).collect(), ks.iter().map(Host::ptr).collect(),
        vs.iter().map(Host::ptr).collect());
    let mut out = Host::zeros(dtype, b * n * hq * d)?;
    let mut m = vec![0f32; b * hq * n];
    let mut l = vec![0f32; b * hq * n];
    check(unsafe {
        lc_ring_fwd_with_stats_host(&dsc, qp.as_ptr(), kp.as_ptr(), vp.as_ptr(), out.mut_ptr(),
                                    m.as_mut_ptr(), l.as_mut_ptr())
    })?;
    Ok((out.tensor(dims)?,
        Tensor::from_vec(m, (b, hq, n, 1), &Device::Cpu)?,
        Tensor::from_vec(l, (b, hq, n, 1), &Device::Cpu)?))
}

/// ring_causal_attention_forward (ring_attention.rs:116-135).
pub fn ring_causal_attention_forward(
    shards: &[(Tensor, Tensor, Tensor)], rank: usize, causal: bool, block_q: usize,
    block_k: usize, valid_length: Option<usize>, q_position_start: Option<usize>,
) -> Result<Tensor> {
    Ok(ring_causal_attention_forward_with_stats(shards, rank, causal, block_q, block_k,
                                                valid_length, q_position_start)?.0)
}

/// ring_causal_attention_backward (ring_attention.rs:281-475) on the GPU: this rank's
/// (dq, dk, dv); dk, dv are summed over each GQA group.
#[allow(clippy::too_many_arguments)]
pub fn ring_causal_attention_backward(
    shards: &[(Tensor, Tensor, Tensor)], rank: usize, outs: &[Tensor], ms: &[Tensor],
    ls: &[Tensor], grad_outs: &[Tensor], causal: bool, block_q: usize, block_k: usize,
    valid_length: Option<usize>, q_position_start: Option<usize>,
) -> Result<(Tensor, Tensor, Tensor)> {
    let (dims, hkv) = shard_dims(shards, rank)?;
    let (b, n, _hq, d) = dims;
    let dtype = shards[rank].0.dtype();
    let dsc = desc(shards.len(), rank, dims, hkv, dtype, causal, block_q, block_k, valid_length,
                   q_position_start)?;
    let host = |ts: Vec<&Tensor>| ts.into_iter().map(Host::of).collect::<Result<Vec<_>>>();
    let qs = host(shards.iter().map(|s| &s.0).collect())?;
    let ks = host(shards.iter().map(|s| &s.1).collect())?;
    let vs = host(shards.iter().map(|s| &s.2).collect())?;
    let os = host(outs.iter().collect())?;
    let gs = host(grad_outs.iter().collect())?;
    let f32v = |ts: &[Tensor]| ts.iter().map(|t| t.flatten_all()?.to_dtype(DType::F32)?
                                               .to_vec1::<f32>()).collect::<Result<Vec<_>>>();
    let (mv, lv) = (f32v(ms)?, f32v(ls)?);
    let p = |h: &Vec<Host>| h.iter().map(Host::ptr).collect::<Vec<_>>();
    let (mp, lp): (Vec<_>, Vec<_>) = (mv.iter().map(|v| v.as_ptr()).collect(),
                                      lv.iter().map(|v| v.as_ptr()).collect());
    let mut dq = Host::zeros(dtype, dims.0 * n * dims.2 * d)?;
    let mut dk = Host::zeros(dtype, b * n * hkv * d)?;
    let mut dv = Host::zeros(dtype, b * n * hkv * d)?;
    check(unsafe {
        lc_ring_bwd_host(&dsc, p(&qs).as_ptr(), p(&ks).as_ptr(), p(&vs).as_ptr(),
                         p(&os).as_ptr(), mp.as_ptr(), lp.as_ptr(), p(&gs).as_ptr(),
                         dq.mut_ptr(), dk.mut_ptr(), dv.mut_ptr())
    })?;
    Ok((dq.tensor(dims)?, dk.tensor((b, n, hkv, d))?, dv.tensor((b, n, hkv, d))?))
}

/// Causal attention of one [B, T, H, D] sequence as a candle op with a custom backward, for
/// the dense block of SelfAttention::forward_impl (model.rs:223-252).  The forward keeps
/// (m, l); `bwd` recomputes P from them on the GPU (lc_ring_bwd_host with one rank).
pub struct CausalAttention {
    stats: Mutex<Option<(Vec<f32>, Vec<f32>)>>,
}

impl CausalAttention {
    pub fn new() -> Self {
        Self { stats: Mutex::new(None) }
    }
}

fn slice_of(s: &CpuStorage, l: &Layout) -> Result<Host> {
    let (o0, o1) = match l.contiguous_offsets() {
        Some(x) => x,
        None => candle_core::bail!("attention inputs must be contiguous"),
    };
    match s {
        CpuStorage::F32(v) => Ok(Host::F32(v[o0..o1].to_vec())),
        CpuStorage::BF16(v) => Ok(Host::Bf16(v[o0..o1].to_vec())),
        _ => candle_core::bail!("unsupported dtype"),
    }
}

impl CustomOp3 for CausalAttention {
    fn name(&self) -> &'static str {
        "lc-causal-attention"
    }

    fn cpu_fwd(&self, s1: &CpuStorage, l1: &Layout, s2: &CpuStorage, l2: &Layout,
               s3: &CpuStorage, l3: &Layout) -> Result<(CpuStorage, Shape)> {
        let dims = l1.shape().dims4()?;
        let (b, t, hq, d) = dims;
        let hkv = l2.shape().dims4()?.2;
        let (q, k, v) = (slice_of(s1, l1)?, slice_of(s2, l2)?, slice_of(s3, l3)?);
        let dtype = s1.dtype();
        let dsc = desc(1, 0, dims, hkv, dtype, true, 64, 128, None, None)?;
        let mut out = Host::zeros(dtype, b * t * hq * d)?;
        let (mut m, mut l) = (vec![0f32; b * hq * t], vec![0f32; b * hq * t]);
        check(unsafe {
            lc_ring_fwd_with_stats_host(&dsc, [q.ptr()].as_ptr(), [k.ptr()].as_ptr(),
                                        [v.ptr()].as_ptr(), out.mut_ptr(), m.as_mut_ptr(),
                                        l.as_mut_ptr())
        })?;
        *self.stats.lock().unwrap() = Some((m, l));
        Ok((out.storage(), Shape::from(dims)))
    }

    fn bwd(&self, q: &Tensor, k: &Tensor, v: &Tensor, res: &Tensor, grad_res: &Tensor)
        -> Result<(Option<Tensor>, Option<Tensor>, Option<Tensor>)> {
        let (m, l) = match self.stats.lock().unwrap().clone() {
            Some(x) => x,
            None => candle_core::bail!("backward before forward"),
        };
        let (b, t, hq, _) = q.dims4()?;
        let ms = [Tensor::from_vec(m, (b, hq, t, 1), &Device::Cpu)?];
        let ls = [Tensor::from_vec(l, (b, hq, t, 1), &Device::Cpu)?];
        let grad = grad_res.contiguous()?.to_dtype(res.dtype())?;
        let (dq, dk, dv) = ring_causal_attention_backward(
            &[(q.clone(), k.clone(), v.clone())], 0, &[res.clone()], &ms, &ls, &[grad], true,
            64, 128, None, None)?;
        Ok((Some(dq), Some(dk), Some(dv)))
    }
}
