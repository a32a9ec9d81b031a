// crates/neuron/src/harness/arch/qwen3_5/hx_moe.rs -- the drop-in MoE block for
// neuron: keeps Qwen3_5MoeBlock's surface (load; Module::forward on a rank-3
// (b, l, hidden) tensor, crates/neuron/src/harness/arch/qwen3_5/moe.rs:55,
// 164-199) and runs the block through libhxmoe.so (crates/hx-moe-sys).
// Compiled inside neuron, next to the block it replaces (it uses neuron's
// TextConfig and quantize_parallel); this repository has no cargo, so the
// file is checked by tests/test_abi.py: every sys:: call names a function the
// sys crate declares, with its argument count.
use anyhow::Context;
use candle_core::quantized::GgmlDType;
use candle_core::{DType, Device, Module, Result, Tensor};
use candle_nn::var_builder::ShardedVarBuilder;
use hx_moe_sys as sys;
use std::ffi::{c_void, CStr};

use super::TextConfig;
use crate::harness::tp::isq::quantize_parallel;

/// ISQ types of the expert projections (Q4_K_M: gate/up Q4K, down Q6K;
/// None keeps the checkpoint dtype).
#[derive(Clone, Copy)]
pub struct HxQuant {
    pub gate_up: Option<GgmlDType>,
    pub down: Option<GgmlDType>,
}

/// One checkpoint tensor as host bytes in a format the library reads.
struct HostTensor {
    dtype: i32,
    bytes: Vec<u8>,
}

impl HostTensor {
    /// Unquantised: bf16 bytes for a bf16 tensor, else f32.
    fn plain(t: &Tensor) -> anyhow::Result<Self> {
        let t = t.flatten_all()?;
        Ok(if t.dtype() == DType::BF16 {
            let v = t.to_vec1::<half::bf16>()?;
            Self { dtype: sys::HX_BF16, bytes: v.iter().flat_map(|x| x.to_bits().to_le_bytes()).collect() }
        } else {
            let v = t.to_dtype(DType::F32)?.to_vec1::<f32>()?;
            Self { dtype: sys::HX_F32, bytes: v.iter().flat_map(|x| x.to_le_bytes()).collect() }
        })
    }

    /// GGUF rows of `q`: the bytes quantize_parallel stores in its QTensor.
    fn gguf(t: &Tensor, q: GgmlDType) -> anyhow::Result<Self> {
        let dtype = match q {
            GgmlDType::Q8_0 => sys::HX_Q8_0,
            GgmlDType::Q4K => sys::HX_Q4_K,
            GgmlDType::Q6K => sys::HX_Q6_K,
            other => anyhow::bail!("hx_moe: no kernel for {other:?} experts"),
        };
        let qt = quantize_parallel(t, q)?;
        Ok(Self { dtype, bytes: qt.data()?.into_owned() })
    }

    fn load(w: &Tensor, q: Option<GgmlDType>) -> anyhow::Result<Self> {
        match q {
            Some(q) => Self::gguf(w, q),
            None => Self::plain(w),
        }
    }

    fn ptr(&self) -> *const c_void {
        self.bytes.as_ptr().cast()
    }
}

/// experts.{e}.{name}.weight for every e, stacked [E, out, in]
/// (tp_qwen3_5.rs:1022-1037 at world size 1).
fn stack_experts(cfg: &TextConfig, vb: &ShardedVarBuilder, name: &str, dims: (usize, usize),
                 q: Option<GgmlDType>) -> anyhow::Result<HostTensor> {
    let experts = vb.pp("experts");
    let mut slices = Vec::with_capacity(cfg.num_experts);
    for e in 0..cfg.num_experts {
        let w = experts.pp(e).pp(name).get(dims, "weight")
            .with_context(|| format!("load expert {e} '{name}'"))?;
        slices.push(w);
    }
    HostTensor::load(&Tensor::stack(&slices, 0)?, q)
}

fn check(rc: i32) -> Result<()> {
    if rc == sys::HX_OK {
        return Ok(());
    }
    let msg = unsafe { CStr::from_ptr(sys::hx_last_error()) }.to_string_lossy().into_owned();
    Err(candle_core::Error::Msg(format!("hx_moe: {msg} (status {rc})")))
}

pub struct HxMoeBlock {
    raw: *mut sys::hx_moe,
    act: DType,
}

// One owner thread drives a block (device_worker/mod.rs:103-111): the handle
// is moved there once. The raw pointer keeps the type !Sync, so &self calls
// (Module::forward) are never concurrent, as the ABI requires.
unsafe impl Send for HxMoeBlock {}

impl HxMoeBlock {
    /// Mirrors Qwen3_5MoeBlock::load (moe.rs:55-112): same config fields, same
    /// checkpoint names. The library validates E, k, I and the GGUF
    /// divisibility with the reference's rules and copies every tensor, so
    /// the host bytes are dropped when this returns.
    pub fn load(cfg: &TextConfig, vb: &ShardedVarBuilder, quant: HxQuant, device: i32) -> anyhow::Result<Self> {
        let (h, i, is) = (cfg.hidden_size, cfg.moe_intermediate_size, cfg.shared_expert_intermediate_size);
        let router = HostTensor::plain(&vb.pp("gate").get((cfg.num_experts, h), "weight")?)?;
        let gate = stack_experts(cfg, vb, "gate_proj", (i, h), quant.gate_up)?;
        let up = stack_experts(cfg, vb, "up_proj", (i, h), quant.gate_up)?;
        let down = stack_experts(cfg, vb, "down_proj", (h, i), quant.down)?;
        let shared = if is > 0 {
            let s = vb.pp("shared_expert");
            Some([
                HostTensor::load(&s.pp("gate_proj").get((is, h), "weight")?, quant.gate_up)?,
                HostTensor::load(&s.pp("up_proj").get((is, h), "weight")?, quant.gate_up)?,
                HostTensor::load(&s.pp("down_proj").get((h, is), "weight")?, quant.down)?,
                HostTensor::plain(&vb.pp("shared_expert_gate").get((1, h), "weight")?)?,
            ])
        } else {
            None
        };
        // (dtype, pointer) of shared tensor k, or (0, NULL) without a shared expert
        let sh = |k: usize| shared.as_ref().map_or((0, std::ptr::null()), |s| (s[k].dtype, s[k].ptr()));
        let act = vb.dtype();
        let c = sys::hx_moe_config {
            hidden_size: h as i32,
            num_experts: cfg.num_experts as i32,
            num_experts_per_tok: cfg.num_experts_per_tok as i32,
            moe_intermediate_size: i as i32,
            shared_expert_intermediate_size: is as i32,
            norm_topk_prob: cfg.norm_topk_prob as i32,
            act_dtype: if act == DType::BF16 { sys::HX_BF16 } else { sys::HX_F32 },
        };
        let w = sys::hx_moe_weights {
            location: sys::HX_HOST,
            router_dtype: router.dtype, router: router.ptr(),
            gate_dtype: gate.dtype, experts_gate: gate.ptr(),
            up_dtype: up.dtype, experts_up: up.ptr(),
            down_dtype: down.dtype, experts_down: down.ptr(),
            shared_gate_dtype: sh(0).0, shared_gate: sh(0).1,
            shared_up_dtype: sh(1).0, shared_up: sh(1).1,
            shared_down_dtype: sh(2).0, shared_down: sh(2).1,
            shared_expert_gate_dtype: sh(3).0, shared_expert_gate: sh(3).1,
        };
        let mut raw = std::ptr::null_mut();
        check(unsafe { sys::hx_moe_create(&c, &w, device, &mut raw) })?;
        Ok(Self { raw, act })
    }
}

impl Module for HxMoeBlock {
    fn forward(&self, xs: &Tensor) -> Result<Tensor> {
        let (b, l, h) = xs.dims3()?;
        let n = b * l;
        let x = xs.to_dtype(self.act)?.flatten_all()?;
        let y = if self.act == DType::BF16 {
            let xv = x.to_vec1::<half::bf16>()?;
            let mut yv = vec![half::bf16::ZERO; n * h];
            check(unsafe {
                sys::hx_moe_forward_host(self.raw, xv.as_ptr().cast(), n as i64, yv.as_mut_ptr().cast(), std::ptr::null())
            })?;
            Tensor::from_vec(yv, (b, l, h), &Device::Cpu)?
        } else {
            let xv = x.to_vec1::<f32>()?;
            let mut yv = vec![0f32; n * h];
            check(unsafe {
                sys::hx_moe_forward_host(self.raw, xv.as_ptr().cast(), n as i64, yv.as_mut_ptr().cast(), std::ptr::null())
            })?;
            Tensor::from_vec(yv, (b, l, h), &Device::Cpu)?
        };
        y.to_device(xs.device())?.to_dtype(xs.dtype())
    }
}

impl Drop for HxMoeBlock {
    fn drop(&mut self) {
        unsafe { sys::hx_moe_destroy(self.raw) };
    }
}
