//! HipModel / HipKVCache: the engine of libqe.so behind the methods of the reference's MetalModel /
//! MetalKVCache (metal_infrence_engine/src/metal_inference.rs:100-316), so that a caller of the
//! Metal engine switches by changing the type names.
//!
//! Errors: `load_model` returns io::Result as MetalModel::load_model does (metal_inference.rs:157);
//! the per-token calls panic on a failed call, as the reference's do on contract violations
//! (a position past the cache, metal_inference.rs:286-291), with the library's message.
//!
//! The reference bench (src/bin/bench.rs:29-67) drives engines through its private `Engine`
//! trait; the GPU engine is added there beside `Metal`:
//!
//! ```ignore
//! struct Hip { model: HipModel, cpu: Model, cache: HipKVCache, max_seq: usize }
//! impl Engine for Hip {
//!     fn reset(&mut self) { self.cache = HipKVCache::new(&self.model, self.max_seq); }
//!     fn step(&mut self, token: u32, pos: usize) -> Vec<f32> { self.model.forward(token, pos, &mut self.cache) }
//!     fn model(&self) -> &Model { &self.cpu } // bench.rs reads tensors and config for the byte formula
//!     fn decode(&mut self, first: u32, start_pos: usize, steps: usize, on_token: &mut dyn FnMut(u32)) {
//!         self.model.decode(first, start_pos, steps, &mut self.cache, on_token);
//!     }
//! }
//! ```
//! (`cpu` is `Model::load_model` of the same file; `HipModel::weight_bytes_per_token` gives the
//! same byte count without it.)

use std::ffi::{c_int, c_void, CStr, CString};
use std::io;
use std::rc::Rc;

use crate::*;

fn last_error() -> String {
    // SAFETY: qe_last_error returns a NUL-terminated string valid until the next call on this thread
    unsafe { CStr::from_ptr(qe_last_error()) }.to_string_lossy().into_owned()
}

fn check(rc: c_int) -> io::Result<()> {
    if rc == QE_OK {
        return Ok(());
    }
    let kind = match rc {
        QE_ERR_IO => io::ErrorKind::NotFound,
        QE_ERR_FORMAT | QE_ERR_TENSOR => io::ErrorKind::InvalidData,
        QE_ERR_POS | QE_ERR_ARG => io::ErrorKind::InvalidInput,
        QE_ERR_UNSUPPORTED => io::ErrorKind::Unsupported,
        _ => io::ErrorKind::Other,
    };
    Err(io::Error::new(kind, format!("qe error {rc}: {}", last_error())))
}

fn must(rc: c_int) {
    if let Err(e) = check(rc) {
        panic!("{e}");
    }
}

// The C model handle, freed when the model and every cache made from it are gone: a cache's
// release waits on the model's stream, so the model must outlive it whatever order the owner
// drops them in (bench.rs's engine structs drop the model field first).
struct ModelHandle(*mut qe_model);

impl Drop for ModelHandle {
    fn drop(&mut self) {
        unsafe { qe_model_free(self.0) }
    }
}

/// The model: weights in one device arena on the current HIP device (MetalModel). Neither it nor
/// its caches are Send: calls on one model must not overlap.
pub struct HipModel {
    h: Rc<ModelHandle>,
    m: *mut qe_model,
    cfg: qe_config,
}

/// One sequence's KV cache and RoPE table, tied to the model it was made from (MetalKVCache).
pub struct HipKVCache {
    kv: *mut qe_kv,
    _model: Rc<ModelHandle>,
    pub max_seq: usize,
}

impl HipModel {
    /// MetalModel::load_model (metal_inference.rs:157-168): the safetensors file and the sibling
    /// config.json.
    pub fn load_model(file: &str) -> io::Result<Self> {
        let path = CString::new(file).map_err(|e| io::Error::new(io::ErrorKind::InvalidInput, e))?;
        let mut m = std::ptr::null_mut();
        check(unsafe { qe_model_load(path.as_ptr(), &mut m) })?;
        let h = Rc::new(ModelHandle(m));
        let mut cfg = qe_config::default();
        check(unsafe { qe_model_config(m, &mut cfg) })?;
        Ok(HipModel { h, m, cfg })
    }

    /// MetalModel::config (metal_inference.rs:170)
    pub fn config(&self) -> &qe_config {
        &self.cfg
    }

    /// bench.rs:106-116: every tensor's bytes except the embedding table, plus one embedding row
    pub fn weight_bytes_per_token(&self) -> usize {
        unsafe { qe_weight_bytes_per_token(self.m) as usize }
    }

    /// bench.rs:118-119: K and V bytes read at position pos with an f32 cache
    pub fn kv_bytes_at(&self, pos: usize) -> usize {
        unsafe { qe_kv_bytes_at(self.m, pos as u64, QE_KV_F32) as usize }
    }

    /// MetalModel::forward (metal_inference.rs:284-291): `token` at `pos`, its K/V into the cache,
    /// the vocab_size logits back.
    pub fn forward(&self, token: u32, pos: usize, cache: &mut HipKVCache) -> Vec<f32> {
        let mut logits = vec![0f32; self.cfg.vocab_size as usize];
        must(unsafe { qe_forward(self.m, token, pos as u64, cache.kv, logits.as_mut_ptr()) });
        logits
    }

    /// MetalModel::decode (metal_inference.rs:293-316): `steps` greedy steps from `first` at
    /// `start_pos`, each step's argmax feeding the next on the device; on_token gets each token in
    /// order as its step finishes.
    pub fn decode(&self, first: u32, start_pos: usize, steps: usize, cache: &mut HipKVCache,
                  on_token: &mut dyn FnMut(u32)) {
        unsafe extern "C" fn trampoline(user: *mut c_void, tok: u32) {
            let f = &mut *(user as *mut &mut dyn FnMut(u32));
            f(tok);
        }
        let mut cb: &mut dyn FnMut(u32) = on_token;
        let user = &mut cb as *mut &mut dyn FnMut(u32) as *mut c_void;
        must(unsafe {
            qe_decode(self.m, first, start_pos as u64, steps as u64, cache.kv, Some(trampoline), user,
                      std::ptr::null_mut())
        });
    }

    /// The prompt loop of bench.rs:174-176 in one call, through the matrix cores in chunks of up
    /// to 512 tokens: the last token's logits (no reference counterpart).
    pub fn prefill(&self, ids: &[u32], start_pos: usize, cache: &mut HipKVCache) -> Vec<f32> {
        let mut logits = vec![0f32; self.cfg.vocab_size as usize];
        must(unsafe {
            qe_prefill_batch(self.m, ids.as_ptr(), ids.len() as u64, start_pos as u64, cache.kv, 0,
                             logits.as_mut_ptr())
        });
        logits
    }

    /// k <= 64 tokens in one pass at start_pos..: row i holds the logits after ids[i]; the cache
    /// keeps all k positions (a caller that accepts j < k continues at start_pos + j + 1).
    pub fn verify(&self, ids: &[u32], start_pos: usize, cache: &mut HipKVCache) -> Vec<Vec<f32>> {
        let v = self.cfg.vocab_size as usize;
        let mut flat = vec![0f32; ids.len() * v];
        must(unsafe {
            qe_verify(self.m, ids.as_ptr(), ids.len() as u64, start_pos as u64, cache.kv, flat.as_mut_ptr())
        });
        flat.chunks(v).map(|r| r.to_vec()).collect()
    }

    /// Greedy decode by prompt lookup: the tokens of `decode`, in fewer passes where the text
    /// repeats (README.md:109-111). `context` is the prompt.
    pub fn decode_lookup(&self, context: &[u32], first: u32, start_pos: usize, steps: usize,
                         cache: &mut HipKVCache, on_token: &mut dyn FnMut(u32)) -> qe_lookup_stats {
        unsafe extern "C" fn trampoline(user: *mut c_void, tok: u32) {
            let f = &mut *(user as *mut &mut dyn FnMut(u32));
            f(tok);
        }
        let mut cb: &mut dyn FnMut(u32) = on_token;
        let user = &mut cb as *mut &mut dyn FnMut(u32) as *mut c_void;
        let mut st = qe_lookup_stats::default();
        must(unsafe {
            qe_decode_lookup(self.m, context.as_ptr(), context.len() as u64, first, start_pos as u64, steps as u64,
                             cache.kv, 4, 3, Some(trampoline), user, &mut st)
        });
        st
    }
}

impl HipKVCache {
    /// MetalKVCache::new (metal_inference.rs:129-137): an f32 cache of max_seq positions.
    pub fn new(model: &HipModel, max_seq: usize) -> Self {
        Self::with_dtype(model, max_seq, QE_KV_F32)
    }

    /// A cache with bf16 K/V elements (QE_KV_BF16; no reference counterpart).
    pub fn with_dtype(model: &HipModel, max_seq: usize, kv_dtype: c_int) -> Self {
        let mut kv = std::ptr::null_mut();
        must(unsafe { qe_kv_new(model.m, max_seq as u64, kv_dtype, &mut kv) });
        HipKVCache { kv, _model: Rc::clone(&model.h), max_seq }
    }

    /// positions cached so far
    pub fn len(&self) -> usize {
        unsafe { qe_kv_len(self.kv) as usize }
    }

    pub fn is_empty(&self) -> bool {
        self.len() == 0
    }
}

impl Drop for HipKVCache {
    fn drop(&mut self) {
        // runs before the `_model` field's drop: the model is still alive here
        unsafe { qe_kv_free(self.kv) }
    }
}
