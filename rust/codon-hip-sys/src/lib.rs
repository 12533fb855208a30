//! Raw FFI of `libcodon_hip.so`, declared one for one from
//! `include/codon_hip.h`, plus a thin safe layer (`Model`, `Decoder`,
//! `Error`) that owns the handles and turns status codes into
//! `std::io::Error`.  The crate has no dependencies; the codon-infer side
//! (`GpuModel`, `forward_bidirectional_gpu`, the `ModelWeightsRef::Gpu` arms)
//! lives in `rust/codon-infer-gpu/gpu.rs`, which uses the crate's own types.
#![allow(non_camel_case_types)]

use std::ffi::{c_char, c_int, c_void, CStr, CString};
use std::io;
use std::ptr;

// ---- status codes and flags (codon_hip.h) ---------------------------------

pub const CIH_OK: c_int = 0;
pub const CIH_ERR_ARG: c_int = -1;
pub const CIH_ERR_SHAPE: c_int = -2;
pub const CIH_ERR_CAPACITY: c_int = -3;
pub const CIH_ERR_CONTACTS: c_int = -4;
pub const CIH_ERR_HIP: c_int = -5;
pub const CIH_ERR_IO: c_int = -6;
pub const CIH_ERR_FORMAT: c_int = -7;
pub const CIH_ERR_TOKEN: c_int = -8;

pub const CIH_DTYPE_FP32: i32 = 0;
pub const CIH_DTYPE_Q8_0: i32 = 1;
pub const CIH_DTYPE_Q4_0: i32 = 2;

pub const CIH_OUT_LOGITS: u32 = 1 << 0;
pub const CIH_OUT_HIDDEN: u32 = 1 << 1;
pub const CIH_OUT_FINAL_ATT: u32 = 1 << 2;
pub const CIH_OUT_CONTACTS: u32 = 1 << 3;
pub const CIH_OUT_ATTN: u32 = 1 << 4;
pub const CIH_OUT_LAYER_HIDDEN: u32 = 1 << 5;
pub const CIH_IO_DEVICE: u32 = 1 << 16;

pub const CIH_DMS_MASKED_MARGINAL: i32 = 0;
pub const CIH_DMS_WILDTYPE_MARGINAL: i32 = 1;

pub const CIH_KC_GEMM_QUANT: i32 = 0;
pub const CIH_KC_GEMM_FP32: i32 = 1;
pub const CIH_KC_ATTENTION: i32 = 2;
pub const CIH_KC_OTHER: i32 = 3;

#[repr(C)]
#[derive(Clone, Copy, Debug, Default)]
pub struct cih_config {
    pub dim: i32,
    pub hidden_dim: i32,
    pub n_layers: i32,
    pub n_heads: i32,
    pub vocab_size: i32,
    pub max_seq_len: i32,
}

/// Host tensors in `EsmWeights` / `EsmWeightsQ8` / `EsmWeightsQ4` field
/// order; quantized matrices point at packed 36 / 20-byte blocks.
#[repr(C)]
pub struct cih_host_weights {
    pub token_embedding_table: *const c_void,
    pub ln_1_weight: *const f32,
    pub ln_1_bias: *const f32,
    pub wq: *const c_void,
    pub bq: *const f32,
    pub wk: *const c_void,
    pub bk: *const f32,
    pub wv: *const c_void,
    pub bv: *const f32,
    pub wo: *const c_void,
    pub bo: *const f32,
    pub ln_2_weight: *const f32,
    pub ln_2_bias: *const f32,
    pub fc1_weight: *const c_void,
    pub fc1_bias: *const f32,
    pub fc2_weight: *const c_void,
    pub fc2_bias: *const f32,
    pub ln_f_weight: *const f32,
    pub ln_f_bias: *const f32,
    pub classifier_weights: *const f32,
    pub classifier_len: i64,
}

#[repr(C)]
pub struct cih_outputs {
    pub logits: *mut f32,
    pub hidden: *mut f32,
    pub final_att: *mut f32,
    pub contacts: *mut f32,
    pub attn: *mut f32,
    pub layer_hidden: *mut f32,
}

impl Default for cih_outputs {
    fn default() -> Self {
        cih_outputs {
            logits: ptr::null_mut(),
            hidden: ptr::null_mut(),
            final_att: ptr::null_mut(),
            contacts: ptr::null_mut(),
            attn: ptr::null_mut(),
            layer_hidden: ptr::null_mut(),
        }
    }
}

#[repr(C)]
#[derive(Clone, Copy, Debug, Default)]
pub struct cih_kernel_stats {
    pub launches: i64,
    pub total_ms: f64,
    pub flops: f64,
    pub bytes: f64,
}

#[repr(C)]
pub struct cih_model {
    _private: [u8; 0],
}

#[repr(C)]
pub struct cih_decoder {
    _private: [u8; 0],
}

extern "C" {
    pub fn cih_model_create(cfg: *const cih_config, dtype: i32, w: *const cih_host_weights, contact_w: *const f32,
                            contact_b: f32, out: *mut *mut cih_model) -> c_int;
    pub fn cih_model_create_from_file(path: *const c_char, quantize_to: i32, contact_w: *const f32, contact_b: f32,
                                      out: *mut *mut cih_model) -> c_int;
    pub fn cih_model_reserve(m: *mut cih_model, max_batch: i32, max_seq_len: i32, flags: u32) -> c_int;
    pub fn cih_model_config(m: *const cih_model, cfg: *mut cih_config, dtype: *mut i32) -> c_int;
    pub fn cih_model_destroy(m: *mut cih_model) -> c_int;

    pub fn cih_forward(m: *mut cih_model, tokens: *const i32, lens: *const i32, b: i32, s_max: i32, flags: u32,
                       out: *const cih_outputs) -> c_int;

    pub fn cih_decoder_create(m: *mut cih_model, n_slots: i32, max_len: i32, max_rows: i32,
                              out: *mut *mut cih_decoder) -> c_int;
    pub fn cih_decoder_destroy(d: *mut cih_decoder) -> c_int;
    pub fn cih_decoder_reset(d: *mut cih_decoder, slot: i32) -> c_int;
    pub fn cih_decode(d: *mut cih_decoder, slots: *const i32, tokens: *const i32, pos: *const i32, n: i32,
                      logits: *mut f32) -> c_int;
    pub fn cih_generate(d: *mut cih_decoder, n: i32, slots: *const i32, prompts: *const i32, offsets: *const i32,
                        temperature: f32, max_new_tokens: i32, seeds: *const u64, max_seq_len: i32,
                        out_tokens: *mut i32, out_cap: i32, n_generated: *mut i32, prefill_ms: *mut f64,
                        generation_ms: *mut f64) -> c_int;

    pub fn cih_dms(m: *mut cih_model, residues: *const i32, n: i32, window: i32, stride: i32, mode: i32, chunk: i32,
                   deltas: *mut f32, entropy: *mut f32) -> c_int;

    pub fn cih_matmul_tiled(dtype: i32, out: *mut f32, x: *const f32, w: *const c_void, bias: *const f32, in_dim: i32,
                            out_dim: i32, seq_len: i32) -> c_int;
    pub fn cih_matmul_tiled_noalloc(dtype: i32, out: *mut f32, x: *const f32, w: *const c_void, bias: *const f32,
                                    in_dim: i32, out_dim: i32, seq_len: i32, stream: *mut c_void) -> c_int;
    pub fn cih_dequantize_device(dtype: i32, blocks: *const c_void, nblocks: i64, out: *mut f32) -> c_int;
    pub fn cih_quantize_device(dtype: i32, src: *const f32, n: i64, dst: *mut c_void) -> c_int;

    pub fn cih_quantize_q8(src: *const f32, n: i64, dst: *mut c_void) -> c_int;
    pub fn cih_quantize_q4(src: *const f32, n: i64, dst: *mut c_void) -> c_int;
    pub fn cih_dequantize_q8(blocks: *const c_void, nblocks: i64, dst: *mut f32) -> c_int;
    pub fn cih_dequantize_q4(blocks: *const c_void, nblocks: i64, dst: *mut f32) -> c_int;
    pub fn cih_tokenize(text: *const c_char, out: *mut i32, cap: i32) -> c_int;
    pub fn cih_log_softmax_canonical(logits: *const f32, out33: *mut f32) -> c_int;

    pub fn cih_profile_enable(m: *mut cih_model, enable: i32) -> c_int;
    pub fn cih_profile_read(m: *const cih_model, kernel_class: i32, out: *mut cih_kernel_stats) -> c_int;

    pub fn cih_last_error() -> *const c_char;
    pub fn cih_abi_version() -> c_int;
}

// ---- safe layer --------------------------------------------------------------

/// The thread's last library error as an `io::Error` (the reference's
/// loaders return `io::Result`, lib.rs:340-345).
pub fn error(rc: c_int) -> io::Error {
    let msg = unsafe { CStr::from_ptr(cih_last_error()) }.to_string_lossy().into_owned();
    let kind = match rc {
        CIH_ERR_IO => io::ErrorKind::NotFound,
        CIH_ERR_FORMAT => io::ErrorKind::InvalidData,
        CIH_ERR_ARG | CIH_ERR_SHAPE | CIH_ERR_TOKEN => io::ErrorKind::InvalidInput,
        _ => io::ErrorKind::Other,
    };
    io::Error::new(kind, format!("codon_hip status {rc}: {msg}"))
}

fn check(rc: c_int) -> io::Result<()> {
    if rc == CIH_OK {
        Ok(())
    } else {
        Err(error(rc))
    }
}

/// A device-resident model and its workspace.  One call at a time: the
/// handle is not re-entrant (callers wrap it in a `Mutex`).
pub struct Model {
    raw: *mut cih_model,
}

unsafe impl Send for Model {}

impl Model {
    /// `cih_model_create` from host tensors in the crate's field order.
    ///
    /// # Safety
    /// Every pointer in `w` must reference a tensor of the size the
    /// configuration implies, valid for the duration of the call.
    pub unsafe fn from_host(cfg: &cih_config, dtype: i32, w: &cih_host_weights, contact: Option<(&[f32], f32)>)
                            -> io::Result<Self> {
        let (cw, cb) = contact.map_or((ptr::null(), 0.0), |(w, b)| (w.as_ptr(), b));
        let mut raw = ptr::null_mut();
        check(cih_model_create(cfg, dtype, w, cw, cb, &mut raw))?;
        Ok(Model { raw })
    }

    /// `cih_model_create_from_file`: CODQ (FP32/Q8_0/Q4_0), grouped_canonical_v1
    /// or sequential_hf; `quantize_to` -1 keeps the file's format.
    pub fn from_file(path: &str, quantize_to: i32, contact: Option<(&[f32], f32)>) -> io::Result<Self> {
        let c = CString::new(path).map_err(|e| io::Error::new(io::ErrorKind::InvalidInput, e))?;
        let (cw, cb) = contact.map_or((ptr::null(), 0.0), |(w, b)| (w.as_ptr(), b));
        let mut raw = ptr::null_mut();
        check(unsafe { cih_model_create_from_file(c.as_ptr(), quantize_to, cw, cb, &mut raw) })?;
        Ok(Model { raw })
    }

    pub fn reserve(&mut self, max_batch: usize, max_seq_len: usize, flags: u32) -> io::Result<()> {
        check(unsafe { cih_model_reserve(self.raw, max_batch as i32, max_seq_len as i32, flags) })
    }

    pub fn config(&self) -> (cih_config, i32) {
        let mut c = cih_config::default();
        let mut dt = 0i32;
        unsafe { cih_model_config(self.raw, &mut c, &mut dt) };
        (c, dt)
    }

    /// One batched forward; `tokens` is `[lens.len()][s_max]`, outputs point
    /// at host buffers of the padded sizes in codon_hip.h.
    ///
    /// # Safety
    /// The output pointers named in `flags` must reference buffers of those sizes.
    pub unsafe fn forward(&mut self, tokens: &[i32], lens: &[i32], s_max: usize, flags: u32, out: &cih_outputs)
                          -> io::Result<()> {
        assert!(tokens.len() >= lens.len() * s_max, "tokens must hold [B][S_max] ids");
        check(cih_forward(self.raw, tokens.as_ptr(), lens.as_ptr(), lens.len() as i32, s_max as i32, flags, out))
    }

    /// The whole in-silico scan of one protein: deltas `[n][20]` in
    /// CANONICAL_AAS order and entropy `[n]`.
    pub fn dms(&mut self, residues: &[i32], window: usize, stride: usize, mode: i32, chunk: usize)
               -> io::Result<(Vec<f32>, Vec<f32>)> {
        let n = residues.len();
        let (mut d, mut e) = (vec![0f32; n * 20], vec![0f32; n]);
        check(unsafe {
            cih_dms(self.raw, residues.as_ptr(), n as i32, window as i32, stride as i32, mode, chunk as i32,
                    d.as_mut_ptr(), e.as_mut_ptr())
        })?;
        Ok((d, e))
    }

    pub fn raw(&self) -> *mut cih_model {
        self.raw
    }
}

impl Drop for Model {
    fn drop(&mut self) {
        unsafe { cih_model_destroy(self.raw) };
    }
}

/// KV-cache slots for autoregressive decoding on a model (shares its stream).
pub struct Decoder {
    raw: *mut cih_decoder,
}

impl Decoder {
    pub fn new(model: &mut Model, n_slots: usize, max_len: usize, max_rows: usize) -> io::Result<Self> {
        let mut raw = ptr::null_mut();
        check(unsafe { cih_decoder_create(model.raw, n_slots as i32, max_len as i32, max_rows as i32, &mut raw) })?;
        Ok(Decoder { raw })
    }

    /// One stream: the prompt ids without the trailing `<eos>`; returns the
    /// generated ids and the prefill / generation times in ms.
    pub fn generate(&mut self, prompt: &[i32], temperature: f32, max_new_tokens: Option<usize>, seed: u64,
                    max_seq_len: usize) -> io::Result<(Vec<i32>, f64, f64)> {
        let cap = max_seq_len.max(1);
        let offs = [0i32, prompt.len() as i32];
        let (mut out, mut n, mut pre, mut gen) = (vec![0i32; cap], 0i32, 0f64, 0f64);
        check(unsafe {
            cih_generate(self.raw, 1, [0i32].as_ptr(), prompt.as_ptr(), offs.as_ptr(), temperature,
                         max_new_tokens.map_or(-1, |v| v as i32), [seed].as_ptr(), max_seq_len as i32,
                         out.as_mut_ptr(), cap as i32, &mut n, &mut pre, &mut gen)
        })?;
        out.truncate(n as usize);
        Ok((out, pre, gen))
    }
}

impl Drop for Decoder {
    fn drop(&mut self) {
        unsafe { cih_decoder_destroy(self.raw) };
    }
}

/// `Tokenizer::encode` (lib.rs:6511-6521) through the library.
pub fn tokenize(text: &str) -> io::Result<Vec<i32>> {
    let c = CString::new(text).map_err(|e| io::Error::new(io::ErrorKind::InvalidInput, e))?;
    let mut out = vec![0i32; text.chars().count() + 2];
    let n = unsafe { cih_tokenize(c.as_ptr(), out.as_mut_ptr(), out.len() as i32) };
    if n < 0 {
        return Err(error(n));
    }
    out.truncate(n as usize);
    Ok(out)
}
