//! `src/gpu.rs` for the codon-infer crate: the GPU arm of every forward.
//!
//! Add `codon-hip-sys = { path = "<repo>/rust/codon-hip-sys" }` to the
//! crate's Cargo.toml, `pub mod gpu;` to src/lib.rs, a `Gpu(&'a gpu::GpuModel)`
//! variant to `ModelWeightsRef` (lib.rs:2264-2269), and at each dispatch site
//! (pipeline.rs:131-148, 179-196, 237-254, 427-444, 629-646, 1305-1322,
//! 1858-1875) the arm
//!
//!     ModelWeightsRef::Gpu(m) => gpu::forward_bidirectional_gpu(&tokens, config, m, &mut state),
//!
//! `forward_bidirectional_gpu` fills the same `BidirectionalRunState` fields
//! the CPU forwards leave behind (lib.rs:5379-5440): `logits`, `x` (after the
//! final LayerNorm), `final_layer_att` and, when `compute_contacts`,
//! `contact_probs` with row stride n = S - 2.  It panics where the reference
//! panics (a sequence longer than `state.max_len`, lib.rs:5106; n > 1024 with
//! contacts, lib.rs:5046).

use std::io;
use std::sync::Mutex;

use codon_hip_sys as sys;

use crate::{BidirectionalRunState, DmsPositionRow, EsmConfig, EsmWeights, EsmWeightsQ4, EsmWeightsQ8, Tokenizer};

/// A device-resident model behind a lock: one forward per handle at a time,
/// as the reference's run_lock serialises its pool (lib.rs:2750).
pub struct GpuModel {
    inner: Mutex<sys::Model>,
    reserved_len: Mutex<usize>,
}

fn sys_config(cfg: &EsmConfig) -> sys::cih_config {
    sys::cih_config {
        dim: cfg.dim as i32,
        hidden_dim: cfg.hidden_dim as i32,
        n_layers: cfg.n_layers as i32,
        n_heads: cfg.n_heads as i32,
        vocab_size: cfg.vocab_size as i32,
        max_seq_len: cfg.max_seq_len as i32,
    }
}

/// Every output a forward may request; reserving them all once lets one
/// handle serve every caller of the crate.
const ALL: u32 = sys::CIH_OUT_LOGITS
    | sys::CIH_OUT_HIDDEN
    | sys::CIH_OUT_FINAL_ATT
    | sys::CIH_OUT_CONTACTS
    | sys::CIH_OUT_LAYER_HIDDEN;

macro_rules! host_weights {
    ($w:expr) => {
        sys::cih_host_weights {
            token_embedding_table: $w.token_embedding_table.as_ptr().cast(),
            ln_1_weight: $w.ln_1_weight.as_ptr(),
            ln_1_bias: $w.ln_1_bias.as_ptr(),
            wq: $w.wq.as_ptr().cast(),
            bq: $w.bq.as_ptr(),
            wk: $w.wk.as_ptr().cast(),
            bk: $w.bk.as_ptr(),
            wv: $w.wv.as_ptr().cast(),
            bv: $w.bv.as_ptr(),
            wo: $w.wo.as_ptr().cast(),
            bo: $w.bo.as_ptr(),
            ln_2_weight: $w.ln_2_weight.as_ptr(),
            ln_2_bias: $w.ln_2_bias.as_ptr(),
            fc1_weight: $w.fc1_weight.as_ptr().cast(),
            fc1_bias: $w.fc1_bias.as_ptr(),
            fc2_weight: $w.fc2_weight.as_ptr().cast(),
            fc2_bias: $w.fc2_bias.as_ptr(),
            ln_f_weight: $w.ln_f_weight.as_ptr(),
            ln_f_bias: $w.ln_f_bias.as_ptr(),
            classifier_weights: $w.classifier_weights.as_ptr(),
            classifier_len: $w.classifier_weights.len() as i64,
        }
    };
}

impl GpuModel {
    fn wrap(mut m: sys::Model, max_len: usize) -> io::Result<Self> {
        m.reserve(1, max_len, ALL)?;
        Ok(GpuModel { inner: Mutex::new(m), reserved_len: Mutex::new(max_len) })
    }

    /// `EsmWeights` (FP32), uploaded once; the caller's vectors may be dropped afterwards.
    pub fn from_fp32(cfg: &EsmConfig, w: &EsmWeights, max_len: usize) -> io::Result<Self> {
        let (cw, cb) = cfg.contact_head_weights();
        let hw = host_weights!(w);
        let m = unsafe { sys::Model::from_host(&sys_config(cfg), sys::CIH_DTYPE_FP32, &hw, Some((&cw[..], cb)))? };
        Self::wrap(m, max_len)
    }

    /// `EsmWeightsQ8`: the `Vec<BlockQ8_0>` buffers go over as packed 36-byte blocks.
    pub fn from_q8(cfg: &EsmConfig, w: &EsmWeightsQ8, max_len: usize) -> io::Result<Self> {
        let (cw, cb) = cfg.contact_head_weights();
        let hw = host_weights!(w);
        let m = unsafe { sys::Model::from_host(&sys_config(cfg), sys::CIH_DTYPE_Q8_0, &hw, Some((&cw[..], cb)))? };
        Self::wrap(m, max_len)
    }

    /// `EsmWeightsQ4`: packed 20-byte `BlockQ4_0` matrices, FP32 embedding.
    pub fn from_q4(cfg: &EsmConfig, w: &EsmWeightsQ4, max_len: usize) -> io::Result<Self> {
        let (cw, cb) = cfg.contact_head_weights();
        let hw = host_weights!(w);
        let m = unsafe { sys::Model::from_host(&sys_config(cfg), sys::CIH_DTYPE_Q4_0, &hw, Some((&cw[..], cb)))? };
        Self::wrap(m, max_len)
    }

    /// `load_model_weights` (main.rs:137-244) straight to the device:
    /// `quantize_to` -1 keeps the file's format, 1 / 2 quantize FP32 to Q8_0 / Q4_0.
    pub fn from_file(path: &str, cfg: &EsmConfig, quantize_to: i32, max_len: usize) -> io::Result<Self> {
        let (cw, cb) = cfg.contact_head_weights();
        let m = sys::Model::from_file(path, quantize_to, Some((&cw[..], cb)))?;
        Self::wrap(m, max_len)
    }

    fn ensure_len(&self, m: &mut sys::Model, s: usize) -> io::Result<()> {
        let mut r = self.reserved_len.lock().unwrap();
        if s > *r {
            m.reserve(1, s, ALL)?;
            *r = s;
        }
        Ok(())
    }
}

/// Same contract as forward_bidirectional_q8 (lib.rs:5442) on a GPU model.
pub fn forward_bidirectional_gpu(tokens: &[usize], config: &EsmConfig, model: &GpuModel,
                                 state: &mut BidirectionalRunState) {
    forward_bidirectional_gpu_ext(tokens, config, model, state, None)
}

/// forward_bidirectional_parallel_ext (lib.rs:5097) on a GPU model: `on_layer`
/// receives each layer's residual stream `[S][dim]` after the layer.
pub fn forward_bidirectional_gpu_ext(tokens: &[usize], config: &EsmConfig, model: &GpuModel,
                                     state: &mut BidirectionalRunState,
                                     mut on_layer: Option<&mut dyn FnMut(usize, &[f32])>) {
    let s = tokens.len();
    assert!(s <= state.max_len, "Sequence length {} exceeds max_len {}", s, state.max_len);
    let n_res = s.saturating_sub(2);
    let contacts = state.compute_contacts && n_res > 0;
    if contacts {
        assert!(n_res <= 1024, "contacts need at most 1024 residues (got {})", n_res);
    }
    let toks: Vec<i32> = tokens.iter().map(|&t| t as i32).collect();
    let lens = [s as i32];
    let mut flags = sys::CIH_OUT_LOGITS | sys::CIH_OUT_HIDDEN | sys::CIH_OUT_FINAL_ATT;
    if contacts {
        flags |= sys::CIH_OUT_CONTACTS;
    }
    let mut layers = Vec::new();
    if on_layer.is_some() {
        flags |= sys::CIH_OUT_LAYER_HIDDEN;
        layers = vec![0f32; config.n_layers * s * config.dim];
    }
    let out = sys::cih_outputs {
        logits: state.logits.as_mut_ptr(),
        hidden: state.x.as_mut_ptr(),
        final_att: state.final_layer_att.as_mut_ptr(),
        contacts: if contacts { state.contact_probs.as_mut_ptr() } else { std::ptr::null_mut() },
        attn: std::ptr::null_mut(),
        layer_hidden: if layers.is_empty() { std::ptr::null_mut() } else { layers.as_mut_ptr() },
    };
    let mut m = model.inner.lock().unwrap();
    model.ensure_len(&mut m, s).unwrap_or_else(|e| panic!("{e}"));
    // the outputs' padded strides equal the sequence's own for one sequence
    unsafe { m.forward(&toks, &lens, s, flags, &out) }.unwrap_or_else(|e| panic!("{e}"));
    drop(m);
    if let Some(cb) = on_layer.as_mut() {
        for l in 0..config.n_layers {
            cb(l, &layers[l * s * config.dim..(l + 1) * s * config.dim]);
        }
    }
}

/// run_pipeline_dms_with_mode's scan (pipeline.rs:76-315) as one call: the
/// windowed masked copies run in batches of `chunk` on the device, and only
/// the 20 deltas and the entropy per position come back.
pub fn dms_rows_gpu(seq: &str, model: &GpuModel, window_size: usize, stride: usize, masked: bool, chunk: usize)
                    -> io::Result<Vec<DmsPositionRow>> {
    let toks = Tokenizer::encode(seq);
    let res: Vec<i32> = toks[1..toks.len() - 1].iter().map(|&t| t as i32).collect();
    let n = res.len();
    let mode = if masked { sys::CIH_DMS_MASKED_MARGINAL } else { sys::CIH_DMS_WILDTYPE_MARGINAL };
    let mut m = model.inner.lock().unwrap();
    let (cfg, _) = m.config();
    let window = if window_size == 0 || n <= window_size { n } else { window_size };
    let window = window.min(cfg.max_seq_len as usize);
    m.reserve(chunk.max(1), window + 2, ALL)?;
    let (deltas, entropy) = m.dms(&res, window_size, stride, mode, chunk)?;
    // the workspace now has the scan's shape; forwards re-reserve on demand
    *model.reserved_len.lock().unwrap() = window + 2;
    let chars: Vec<char> = seq.chars().collect();
    Ok((0..n)
        .map(|p| {
            let mut d = [0f32; 20];
            d.copy_from_slice(&deltas[p * 20..p * 20 + 20]);
            DmsPositionRow::new(p + 1, chars[p], d, entropy[p])
        })
        .collect())
}
