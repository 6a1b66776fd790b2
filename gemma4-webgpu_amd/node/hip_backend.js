'use strict';
// HipBackend: the decode step of the reference's WebGPU engine, dispatched key
// by key on libg4hip through the N-API addon g4hip.node, for a Node host.
//
// Written in ES2019 (plain classes and functions, no TypeScript compiler);
// device buffers are the addon's BigInt handles. The pass order, the
// buffers each key binds and its Params follow
//   src/engine.ts:1466-1651  encodeTransformerPass (embed, 35 layers, final norm)
//   src/engine.ts:1670-1746  sampleNextTokenSubmit (LM head, softcap, argmax /
//                            top-k, the sampled token fed to the next embed)
// with the work-buffer names of src/types.ts:489-517 and the layer tensor
// names of the GGUF (attn_q, ffn_down, ...), including the per-layer-embedding
// passes (ple1.* before the layers, src/engine.ts:1516-1535; ple2.* at the end
// of each layer, src/engine.ts:1608-1616).
//
// Differences from the WebGPU backend, all at the boundary:
//  - matrices are the raw GGUF block bytes in the file's own format per
//    tensor (Q4_K or Q6_K: a Q4_K_M file mixes both) rather than f16 rows;
//    the f16 token table is still bound for the embedding lookup, and the
//    per-layer-embedding table stays in its Q5_K blocks (one 256-value block
//    per token and layer), the stage-1 pass dispatching every layer at once;
//  - the KV caches are f16 (2 bytes per element);
//  - dynamic fields (position, seq_len, token) are call arguments or, with a
//    device position / token buffer, read by the kernels themselves, so a
//    whole forward can be captured once (graphBegin/graphEnd) and replayed.

const path = require('path');

function loadAddon() {
  return require(path.join(__dirname, 'g4hip.node'));
}

// computeKvProducerMap (src/config/gemma4-e2b.ts:159-180): a layer past the
// unshared ones reads the cache of the last unshared layer of its kind.
function kvProducerMap(numLayers, numUnshared, isSliding) {
  let lastLocal = -1;
  let lastGlobal = -1;
  for (let i = 0; i < numUnshared; i++) {
    if (isSliding[i]) lastLocal = i;
    else lastGlobal = i;
  }
  const out = [];
  for (let i = 0; i < numLayers; i++) {
    if (i < numUnshared) out.push(i);
    else out.push(isSliding[i] ? lastLocal : lastGlobal);
  }
  return out;
}

// The Gemma-4-E2B configuration (src/config/gemma4-e2b.ts:16-63); any field
// may be overridden (a smaller model for tests: num_layers, num_unshared_layers,
// global_layers, vocab_size, ...).
function e2bConfig(overrides) {
  const o = overrides || {};
  const numLayers = o.num_layers !== undefined ? o.num_layers : 35;
  const globals = o.global_layers || [4, 9, 14, 19, 24, 29, 34];
  const numUnshared = o.num_unshared_layers !== undefined ? o.num_unshared_layers : 15;
  const isSliding = [];
  const inter = [];
  for (let i = 0; i < numLayers; i++) {
    isSliding.push(globals.indexOf(i) < 0);
    inter.push(i < numUnshared ? (o.intermediate_unshared || 6144) : (o.intermediate_shared || 12288));
  }
  return {
    hidden_size: o.hidden_size || 1536,
    num_q_heads: o.num_q_heads || 8,
    num_kv_heads: o.num_kv_heads || 1,
    head_dim_local: o.head_dim_local || 256,
    head_dim_global: o.head_dim_global || 512,
    vocab_size: o.vocab_size || 262144,
    num_layers: numLayers,
    rms_norm_eps: o.rms_norm_eps || 1e-6,
    rope_theta_global: o.rope_theta_global || 1e6,
    rope_theta_swa: o.rope_theta_swa || 1e4,
    sliding_window: o.sliding_window || 512,
    attention_is_sliding: isSliding,
    intermediate_sizes: inter,
    num_unshared_layers: numUnshared,
    kv_producer_for_layer: kvProducerMap(numLayers, numUnshared, isSliding),
    per_layer_input_dim: o.per_layer_input_dim !== undefined ? o.per_layer_input_dim : 256,
    final_logit_softcapping: o.final_logit_softcapping !== undefined ? o.final_logit_softcapping : 30.0,
  };
}

// configFromGGUF (src/config/gemma4-e2b.ts:70-148): the E2B baseline,
// overridden by every gemma4.* key of the file's metadata (ggufMetadata:
// {key: {type, value}}, arrays as lists of {type, value}).
function configFromGGUF(kv, maxContextLength) {
  if (!kv['gemma4.block_count'] && !kv['gemma4.embedding_length']) {
    throw new Error('Not a Gemma 4 GGUF: no gemma4.* metadata keys found.');
  }
  const num = (k) => {
    const e = kv[k];
    if (!e || e.type === 'array' || e.value === null || e.value === undefined) return null;
    return Number(e.value);
  };
  const arr = (k) => {
    const e = kv[k];
    return e && e.type === 'array' && e.value ? e.value.map((x) => x.value) : null;
  };
  const base = e2bConfig();
  const C = Object.assign({}, base);
  const set = (k, field) => {
    const v = num(k);
    if (v !== null) C[field] = v;
  };
  set('gemma4.embedding_length', 'hidden_size');
  set('gemma4.block_count', 'num_layers');
  set('gemma4.attention.head_count', 'num_q_heads');
  set('gemma4.attention.head_count_kv', 'num_kv_heads');
  const ctxLen = num('gemma4.context_length');
  C.context_length = ctxLen !== null ? Math.min(ctxLen, maxContextLength || 2048) : 2048;
  const ffn = arr('gemma4.feed_forward_length');
  if (ffn) {
    C.intermediate_sizes = ffn.map(Number);
  } else {
    const v = num('gemma4.feed_forward_length');
    if (v !== null) C.intermediate_sizes = new Array(C.num_layers).fill(v);
  }
  set('gemma4.attention.key_length', 'head_dim_global');
  set('gemma4.attention.key_length_swa', 'head_dim_local');
  set('gemma4.rope.freq_base', 'rope_theta_global');
  set('gemma4.rope.freq_base_swa', 'rope_theta_swa');
  set('gemma4.attention.sliding_window', 'sliding_window');
  const pat = arr('gemma4.attention.sliding_window_pattern');
  if (pat) C.attention_is_sliding = pat.map(Boolean);
  set('gemma4.embedding_length_per_layer_input', 'per_layer_input_dim');
  set('gemma4.final_logit_softcapping', 'final_logit_softcapping');
  const shared = num('gemma4.attention.shared_kv_layers');
  if (shared !== null) C.num_unshared_layers = C.num_layers - shared;
  C.kv_producer_for_layer = kvProducerMap(C.num_layers, C.num_unshared_layers, C.attention_is_sliding);
  return C;
}

// Per-layer selectors (src/types.ts:69-91).
const isSwaLayer = (C, il) => C.attention_is_sliding[il];
const ropeTheta = (C, il) => (isSwaLayer(C, il) ? C.rope_theta_swa : C.rope_theta_global);
const headDim = (C, il) => (isSwaLayer(C, il) ? C.head_dim_local : C.head_dim_global);
const intermediateSize = (C, il) => C.intermediate_sizes[il];
const isKvProducer = (C, il) => C.kv_producer_for_layer[il] === il;

const LAYER_TENSORS = ['attn_norm', 'attn_q', 'attn_k', 'attn_v', 'attn_q_norm', 'attn_k_norm', 'attn_output',
  'post_attention_norm', 'ffn_norm', 'ffn_gate', 'ffn_up', 'ffn_down', 'post_ffw_norm'];
// per-layer-embedding tensors of a layer (f16), src/engine.ts:63-69
const PLE_TENSORS = ['inp_gate', 'proj', 'post_norm', 'layer_output_scale'];
// the matrices' block formats unless a layer says otherwise
const DEFAULT_FORMATS = { attn_q: 'q4k', attn_k: 'q4k', attn_v: 'q4k', attn_output: 'q4k', ffn_gate: 'q4k',
  ffn_up: 'q4k', ffn_down: 'q6k' };
// bytes per 256 values: Q4_K / Q6_K blocks, or f16 rows
const BLOCK_BYTES = { q4k: 144, q6k: 210, f16: 512 };

class HipBackend {
  // addon: the g4hip.node exports (or any object with the same functions);
  // ctx: its context handle. opts.maxSeqLen (default 2048, the reference's
  // context cap), opts.mr4ForFfn (gate/up through matmulQuantMR4, default
  // true), opts.trace (an array that receives [passLabel, key] per dispatch).
  constructor(addon, ctx, config, opts) {
    const o = opts || {};
    this.g = addon;
    this.ctx = ctx;
    this.config = config;
    this.maxSeqLen = o.maxSeqLen || 2048;
    this.mr4ForFfn = o.mr4ForFfn !== undefined ? o.mr4ForFfn : true;
    this.trace = o.trace || null;
    this.owned = [];
    this.layers = [];      // per layer: {tensor name: handle}
    this.formats = [];     // per layer: {matrix name: 'q4k' | 'q6k' | 'f16'}
    this.globals = {};     // tokenEmbed (f16), lmHead (+ lmHeadFormat), finalNorm, rope_freqs,
                           // perLayerModelProj / perLayerProjNorm (f16), perLayerTable (Q5_K)
    this.workBuffers = {};
    this.kvCaches = [];    // per layer: {k, v} (consumers hold their producer's)
  }

  static open(config, opts) {
    const addon = loadAddon();
    const ctx = addon.init((opts && opts.device) || 0);
    return new HipBackend(addon, ctx, config, opts);
  }

  // A backend holding a GGUF file's weights (GGUFParser + the upload of
  // src/engine.ts:547-625): each layer matrix as the file's Q4_K / Q6_K
  // blocks, and a matrix in another format (F32, F16, BF16, Q5_K, Q8_0) as
  // the reference's f16 rows (tensorToF16, src/engine.ts:570-579); norms and
  // the per-layer-embedding matrices as f16, the tied token table as the LM
  // head's blocks (or rows) and the lookup's f16 rows, the per-layer table as
  // its Q5_K blocks. opts as the constructor's, plus device and
  // maxContextLength.
  static fromGGUF(file, opts) {
    const o = opts || {};
    const addon = loadAddon();
    const gg = addon.ggufOpen(file);
    try {
      const C = configFromGGUF(addon.ggufMetadata(gg), o.maxContextLength);
      const tensors = {};
      for (const t of addon.ggufTensors(gg)) tensors[t.name] = t;
      const emb = tensors['token_embd.weight'];
      if (!emb) throw new Error('GGUF has no token_embd.weight');
      C.vocab_size = emb.dims[1];
      if (!tensors['per_layer_token_embd.weight']) C.per_layer_input_dim = 0;
      const ctx = addon.init(o.device || 0);
      const be = new HipBackend(addon, ctx, C, Object.assign({ maxSeqLen: C.context_length }, o));
      be.allocate();
      be._loadGGUF(gg, tensors);
      return be;
    } finally {
      addon.ggufClose(gg);
    }
  }

  _loadGGUF(gg, tensors) {
    const C = this.config;
    const g = this.g;
    const FMT = { 12: 'q4k', 14: 'q6k' };
    const get = (name) => {
      const t = tensors[name];
      if (!t) throw new Error('GGUF has no tensor ' + name);
      return t;
    };
    const raw = (name) => {
      const t = get(name);
      if (!t.nbytes) throw new Error(name + ': tensor type ' + t.type + ' has no known size');
      const p = this.alloc(t.nbytes);
      g.ggufUpload(this.ctx, gg, t.index, p, t.nbytes);
      return p;
    };
    const f16 = (name) => {
      const t = get(name);
      let n = 1;
      for (const d of t.dims) n *= d;
      const p = this.alloc(2 * Math.max(n, 2));
      g.ggufUploadF16(this.ctx, gg, t.index, p, Math.max(n, 2));
      return p;
    };
    // GGUF types held as f16 rows: F32, F16, BF16 converted on upload;
    // Q8_0 and Q5_K dequantized on the device
    const ROWS = { 0: null, 1: null, 30: null, 8: ['q8_0', 32], 13: ['q5k', 256] };
    const matFormat = (name) => {
      const ty = get(name).type;
      if (FMT[ty]) return FMT[ty];
      if (ROWS[ty] !== undefined) return 'f16';
      throw new Error(name + ': tensor type ' + ty + ' (Q4_K, Q6_K, Q5_K, Q8_0, F16, BF16 or F32 matrices)');
    };
    const matrix = (name) => {
      const t = get(name);
      if (FMT[t.type]) return raw(name);
      const dq = ROWS[t.type];
      if (dq === undefined) matFormat(name);  // throws
      if (dq === null) return f16(name);
      let n = 1;
      for (const d of t.dims) n *= d;
      const tmp = g.alloc(this.ctx, t.nbytes);
      try {
        g.ggufUpload(this.ctx, gg, t.index, tmp, t.nbytes);
        const p = this.alloc(2 * n);
        g.dequantF16(this.ctx, dq[0], tmp, n / dq[1], p);
        g.sync(this.ctx);
        return p;
      } finally {
        g.free(this.ctx, tmp);
      }
    };
    const MATS = ['attn_q', 'attn_k', 'attn_v', 'attn_output', 'ffn_gate', 'ffn_up', 'ffn_down'];
    const F16S = ['attn_norm', 'attn_q_norm', 'attn_k_norm', 'post_attention_norm', 'ffn_norm', 'post_ffw_norm',
      'inp_gate', 'proj', 'post_norm', 'layer_output_scale'];
    for (let il = 0; il < C.num_layers; il++) {
      const prefix = 'blk.' + il + '.';
      const formats = {};
      for (const m of MATS) {
        if (tensors[prefix + m + '.weight'] && (isKvProducer(C, il) || (m !== 'attn_k' && m !== 'attn_v'))) {
          formats[m] = matFormat(prefix + m + '.weight');
        }
      }
      const need = Object.keys(this.layerTensorBytes(il, formats));
      const t = {};
      for (const name of need) {
        t[name] = F16S.indexOf(name) >= 0 ? f16(prefix + name + '.weight') : matrix(prefix + name + '.weight');
      }
      this.setLayerWeights(il, t, formats);
    }
    const glob = { finalNorm: f16('output_norm.weight'), rope_freqs: f16('rope_freqs.weight') };
    const headName = tensors['output.weight'] ? 'output.weight' : 'token_embd.weight';
    glob.lmHead = matrix(headName);
    glob.lmHeadFormat = matFormat(headName);
    // the tied table's f16 rows for the lookup, from the same blocks (or rows)
    const te = headName === 'token_embd.weight' ? glob.lmHead : matrix('token_embd.weight');
    const teFormat = matFormat('token_embd.weight');
    if (teFormat === 'f16') {
      glob.tokenEmbed = te;
    } else {
      glob.tokenEmbed = this.alloc(2 * C.vocab_size * C.hidden_size);
      g.dequantF16(this.ctx, teFormat, te, C.vocab_size * C.hidden_size / 256, glob.tokenEmbed);
    }
    if (C.per_layer_input_dim > 0) {
      glob.perLayerModelProj = f16('per_layer_model_proj.weight');
      glob.perLayerProjNorm = f16('per_layer_proj_norm.weight');
      const ple = get('per_layer_token_embd.weight');
      if (ple.type !== 13) throw new Error('per_layer_token_embd.weight: type ' + ple.type + ', expected Q5_K');
      glob.perLayerTable = raw('per_layer_token_embd.weight');
    }
    this.setGlobals(glob);
    g.sync(this.ctx);
  }

  close() {
    if (this.fusedGraph) {
      this.g.graphDestroy(this.fusedGraph);
      this.fusedGraph = null;
    }
    this._freeBatch();
    for (const p of this.owned) this.g.free(this.ctx, p);
    this.owned = [];
    this.g.destroy(this.ctx);
  }

  alloc(bytes) {
    const p = this.g.alloc(this.ctx, bytes);
    this.owned.push(p);
    return p;
  }

  // Work buffers (src/engine.ts:1001-1064; src/types.ts:489-517) and the f16
  // KV caches of the producer layers.
  allocate() {
    const C = this.config;
    const H = C.hidden_size;
    let maxHd = 0;
    let maxI = 0;
    for (let il = 0; il < C.num_layers; il++) {
      maxHd = Math.max(maxHd, headDim(C, il));
      maxI = Math.max(maxI, intermediateSize(C, il));
    }
    const Q = C.num_q_heads * maxHd;
    const KV = C.num_kv_heads * maxHd;
    const f4 = (n) => this.alloc(4 * n);
    this.workBuffers = {
      hidden: f4(H), residual: f4(H), normed: f4(H), q: f4(Q), k: f4(KV), v: f4(KV), attnOut: f4(Q),
      attnProj: f4(H), attnScores: f4(C.num_q_heads * this.maxSeqLen), ffnGate: f4(maxI), ffnUp: f4(maxI),
      ffnMul: f4(maxI), ffnDown: f4(H), logits: f4(C.vocab_size), argmaxResult: f4(1), topk256Result: f4(512),
      position: f4(1),
    };
    const D = C.per_layer_input_dim;
    if (D > 0) {
      Object.assign(this.workBuffers, { plePmProjected: f4(C.num_layers * D), pleInputs: f4(C.num_layers * D),
        pleGate: f4(D), pleGated: f4(D), pleProjOut: f4(H), plePostNormed: f4(H) });
    }
    this.g.memset(this.ctx, this.workBuffers.argmaxResult, 0, 4);
    this.g.memset(this.ctx, this.workBuffers.position, 0, 4);
    this.kvCaches = [];
    for (let il = 0; il < C.num_layers; il++) {
      if (C.kv_producer_for_layer[il] < 0) throw new Error('layer ' + il + ': no unshared layer of its attention kind');
      if (isKvProducer(C, il)) {
        // rows rounded up to whole pages of 16, so that the batched prefill's
        // paged keys address the same cache through an identity page table
        const bytes = 2 * Math.ceil(this.maxSeqLen / 16) * 16 * C.num_kv_heads * headDim(C, il);
        const kv = { k: this.alloc(bytes), v: this.alloc(bytes) };
        this.g.memset(this.ctx, kv.k, 0, bytes);
        this.g.memset(this.ctx, kv.v, 0, bytes);
        this.kvCaches.push(kv);
      } else {
        this.kvCaches.push(this.kvCaches[C.kv_producer_for_layer[il]]);
      }
    }
  }

  // Byte sizes of a layer's tensors (raw GGUF blocks in `formats`, f16 norm
  // and per-layer-embedding weights).
  layerTensorBytes(il, formats) {
    const C = this.config;
    const F = Object.assign({}, DEFAULT_FORMATS, formats || this.formats[il] || {});
    const H = C.hidden_size;
    const hd = headDim(C, il);
    const Q = C.num_q_heads * hd;
    const KV = C.num_kv_heads * hd;
    const I = intermediateSize(C, il);
    const D = C.per_layer_input_dim;
    const mat = (name, m, n) => (m * n / 256) * BLOCK_BYTES[F[name]];
    const out = {
      attn_norm: 2 * H, attn_q: mat('attn_q', Q, H), attn_q_norm: 2 * hd, attn_output: mat('attn_output', H, Q),
      post_attention_norm: 2 * H, ffn_norm: 2 * H, ffn_gate: mat('ffn_gate', I, H), ffn_up: mat('ffn_up', I, H),
      ffn_down: mat('ffn_down', H, I), post_ffw_norm: 2 * H,
    };
    if (isKvProducer(C, il)) {
      out.attn_k = mat('attn_k', KV, H);
      out.attn_v = mat('attn_v', KV, H);
      out.attn_k_norm = 2 * hd;
    }
    if (D > 0) Object.assign(out, { inp_gate: 2 * D * H, proj: 2 * H * D, post_norm: 2 * H, layer_output_scale: 2 });
    return out;
  }

  // formats: the block format of each matrix that is not the default
  // (Q4_K, ffn_down Q6_K), e.g. {attn_v: 'q6k', ffn_down: 'q4k'}.
  setLayerWeights(il, tensors, formats) {
    const F = Object.assign({}, DEFAULT_FORMATS, formats || {});
    for (const name of Object.keys(F)) {
      if (BLOCK_BYTES[F[name]] === undefined) throw new Error('layer ' + il + ': ' + name + ' format ' + F[name]);
    }
    const need = Object.keys(this.layerTensorBytes(il, F));
    for (const name of need) {
      if (tensors[name] === undefined) throw new Error('layer ' + il + ': missing tensor ' + name);
    }
    this.layers[il] = tensors;
    this.formats[il] = F;
  }

  setGlobals(g) {
    const need = ['tokenEmbed', 'lmHead', 'finalNorm', 'rope_freqs'];
    if (this.config.per_layer_input_dim > 0) need.push('perLayerModelProj', 'perLayerProjNorm', 'perLayerTable');
    for (const name of need) {
      if (g[name] === undefined) throw new Error('missing global ' + name);
    }
    if (g.lmHeadFormat !== undefined && BLOCK_BYTES[g.lmHeadFormat] === undefined) {
      throw new Error('lmHead format ' + g.lmHeadFormat);
    }
    this.globals = g;
  }

  // k, v: [maxSeqLen rounded up to a multiple of 16][num_kv_heads][head_dim] f16
  setKvCache(il, k, v) {
    this.kvCaches[il] = { k: k, v: v };
  }

  _key(label, key) {
    if (this.trace) this.trace.push([label, key]);
  }

  // The WebGPU engine's encodeTransformerPass for `position`. tokenId null:
  // the embedding lookup reads the token the previous sample left on the
  // device (src/engine.ts:1724-1727). positionDev true: position / seq_len
  // are read from the device position counter, which sampleNextToken then
  // advances (so the pass and the sample can be captured once and replayed).
  encodeTransformerPass(tokenId, position, positionDev) {
    const C = this.config;
    const g = this.g;
    const c = this.ctx;
    const W = this.workBuffers;
    const H = C.hidden_size;
    const NQH = C.num_q_heads;
    const NKH = C.num_kv_heads;
    const eps = C.rms_norm_eps;
    const seqLen = position + 1;
    const pd = positionDev ? W.position : null;
    const G = this.globals;

    const tokDev = tokenId === null ? W.argmaxResult : null;
    this._key('embed', 'embeddingLookup');
    g.embeddingLookup(c, G.tokenEmbed, C.vocab_size, W.hidden,
      { hidden_size: H, token_id: tokenId === null ? 0 : tokenId }, tokDev);

    const D = C.per_layer_input_dim;
    if (D > 0) {
      // PLE stage 1: per_layer_model_proj . embedding, then every layer's
      // norm + table row + blend
      this._key('ple1.pmProj', 'matmulQuant');
      g.matmulQuant(c, W.hidden, G.perLayerModelProj, W.plePmProjected, { M: C.num_layers * D, N: H }, 'f16');
      this._key('ple1.stage1Fuse', 'pleStage1Fuse');
      g.pleStage1Fuse(c, W.plePmProjected, G.perLayerProjNorm, G.perLayerTable, C.vocab_size, W.pleInputs,
        { num_layers: C.num_layers, per_layer_dim: D, eps: eps, token_id: tokenId === null ? 0 : tokenId }, tokDev);
    }

    for (let il = 0; il < C.num_layers; il++) {
      const L = this.layers[il];
      const F = this.formats[il] || DEFAULT_FORMATS;
      const HD = headDim(C, il);
      const I = intermediateSize(C, il);
      const Q = NQH * HD;
      const KV = NKH * HD;
      const prod = isKvProducer(C, il);
      const kv = this.kvCaches[C.kv_producer_for_layer[il]];
      const own = this.kvCaches[il];
      const theta = ropeTheta(C, il);
      const applyDivisor = isSwaLayer(C, il) ? 0 : 1;
      const window = isSwaLayer(C, il) ? C.sliding_window : 0;
      // the caller's seq_len (or, from the device, the maximum the scores rows allow)
      const sl = positionDev ? this.maxSeqLen : seqLen;

      this._key('attn.rmsNorm', 'rmsNorm');
      g.rmsNorm(c, W.hidden, L.attn_norm, W.normed, { hidden_size: H, eps: eps });
      const lin = prod ? 'attn.linearQKV.producer' : 'attn.linearQ.consumer';
      this._key(lin, 'matmulQuant');
      g.matmulQuant(c, W.normed, L.attn_q, W.q, { M: Q, N: H }, F.attn_q);
      if (prod) {
        this._key(lin, 'matmulQuant');
        g.matmulQuant(c, W.normed, L.attn_k, W.k, { M: KV, N: H }, F.attn_k);
        this._key(lin, 'matmulQuant');
        g.matmulQuant(c, W.normed, L.attn_v, W.v, { M: KV, N: H }, F.attn_v);
        this._key('attn.vNorm', 'perHeadRmsNormNoWeight');
        g.perHeadRmsNormNoWeight(c, W.v, { num_heads: NKH, head_dim: HD, eps: eps });
      }
      const rope = prod ? 'attn.fusedNormRopeQK' : 'attn.fusedNormRopeQ';
      const rp = (nh) => ({ num_heads: nh, head_dim: HD, eps: eps, position: position, theta: theta,
        apply_divisor: applyDivisor });
      this._key(rope, 'fusedPerHeadNormRope');
      g.fusedPerHeadNormRope(c, W.q, L.attn_q_norm, rp(NQH), G.rope_freqs, pd);
      if (prod) {
        this._key(rope, 'fusedPerHeadNormRope');
        g.fusedPerHeadNormRope(c, W.k, L.attn_k_norm, rp(NKH), G.rope_freqs, pd);
        this._key('attn.kvCacheStore', 'kvCacheStore');
        g.kvCacheStore(c, W.k, W.v, own.k, own.v,
          { num_kv_heads: NKH, head_dim: HD, position: position, max_seq_len: this.maxSeqLen }, pd);
      }
      this._key('attn.attnScore', 'attnScore');
      g.attnScore(c, W.q, kv.k, W.attnScores, { num_q_heads: NQH, num_kv_heads: NKH, head_dim: HD, seq_len: sl,
        scale: 1.0, sliding_window: window }, pd);
      this._key('attn.softmax', 'softmax');
      g.softmax(c, W.attnScores, { num_heads: NQH, seq_len: sl }, pd);
      this._key('attn.attnOutput', 'attnOutput');
      g.attnOutput(c, W.attnScores, kv.v, W.attnOut, { num_q_heads: NQH, num_kv_heads: NKH, head_dim: HD,
        seq_len: sl }, pd);
      this._key('attn.linearOut', 'matmulQuant');
      g.matmulQuant(c, W.attnOut, L.attn_output, W.attnProj, { M: H, N: Q }, F.attn_output);
      this._key('attn.postNormAdd', 'fusedNormAdd');
      g.fusedNormAdd(c, W.attnProj, L.post_attention_norm, W.hidden, W.residual, { size: H, eps: eps });
      this._key('ffn.rmsNorm', 'rmsNorm');
      g.rmsNorm(c, W.residual, L.ffn_norm, W.normed, { hidden_size: H, eps: eps });
      // (the 4-row kernel reads Q4_K only)
      const mm = this.mr4ForFfn && F.ffn_gate === 'q4k' && F.ffn_up === 'q4k' ? 'matmulQuantMR4' : 'matmulQuant';
      this._key('ffn.linearGateUp', mm);
      g[mm](c, W.normed, L.ffn_gate, W.ffnGate, { M: I, N: H }, F.ffn_gate);
      this._key('ffn.linearGateUp', mm);
      g[mm](c, W.normed, L.ffn_up, W.ffnUp, { M: I, N: H }, F.ffn_up);
      this._key('ffn.geluMul', 'geluMul');
      g.geluMul(c, W.ffnGate, W.ffnUp, W.ffnMul, I);
      this._key('ffn.linearDown', 'matmulQuant');
      g.matmulQuant(c, W.ffnMul, L.ffn_down, W.ffnDown, { M: H, N: I }, F.ffn_down);
      this._key('ffn.postNormAdd', 'fusedNormAdd');
      g.fusedNormAdd(c, W.ffnDown, L.post_ffw_norm, W.residual, W.hidden, { size: H, eps: eps });

      if (D > 0) {
        // PLE stage 2 and layer_output_scale
        this._key('ple2.linearInpGate', 'matmulQuant');
        g.matmulQuant(c, W.hidden, L.inp_gate, W.pleGate, { M: D, N: H }, 'f16');
        this._key('ple2.geluMul', 'pleGeluMul');
        g.pleGeluMul(c, W.pleGate, W.pleInputs, W.pleGated, { layer_offset: il * D, size: D });
        this._key('ple2.linearPostProj', 'matmulQuant');
        g.matmulQuant(c, W.pleGated, L.proj, W.pleProjOut, { M: H, N: D }, 'f16');
        this._key('ple2.rmsNorm', 'rmsNorm');
        g.rmsNorm(c, W.pleProjOut, L.post_norm, W.plePostNormed, { hidden_size: H, eps: eps });
        this._key('ple2.skipScaleAdd', 'pleSkipScaleAdd');
        g.pleSkipScaleAdd(c, W.hidden, W.plePostNormed, L.layer_output_scale, { size: H });
      }
    }
    this._key('final.rmsNorm', 'rmsNorm');
    g.rmsNorm(c, W.hidden, G.finalNorm, W.normed, { hidden_size: H, eps: eps });
  }

  // sampleNextTokenSubmit's GPU part: LM head, softcap, then argmax (greedy;
  // the token stays in argmaxResult for the next embed) or top-k 256. With
  // positionDev the device position counter is advanced by one.
  sampleNextToken(greedy, positionDev) {
    const C = this.config;
    const g = this.g;
    const c = this.ctx;
    const W = this.workBuffers;
    const V = C.vocab_size;
    this._key('lmHead', 'matmulQuant');
    g.matmulQuant(c, W.normed, this.globals.lmHead, W.logits, { M: V, N: C.hidden_size },
      this.globals.lmHeadFormat || 'q6k');
    if (C.final_logit_softcapping > 0) {
      this._key('logitSoftcap', 'logitSoftcap');
      g.logitSoftcap(c, W.logits, { size: V, cap: C.final_logit_softcapping });
    }
    if (greedy === false) {
      this._key('sample.topk256', 'topk256');
      g.topk256(c, W.logits, W.topk256Result, V);
    } else {
      this._key('sample.argmax', 'argmax');
      g.argmax(c, W.logits, W.argmaxResult, V);
    }
    if (positionDev) g.advancePosition(c, W.position, 1);
  }

  // ---- the MI355X decode step -------------------------------------------
  // The fused launch sequence of g4hip/decoder.py Decoder.step_fused (greedy
  // sampling): per layer a q/k/v launch per weight format that also forms
  // the layer's normalised input (the previous layer's post-FFN or
  // per-layer-embedding tail as its prologue), the attention block in one
  // launch (q/k norm + RoPE from a per-position table, v norm, KV row store,
  // split-K attention and merge), o, gate/up + GELU (writing the product as
  // the digit block a Q6_K down launch reads), down, and with per-layer
  // embeddings the gate (post-FFN norm-add prologue, GELU x ple epilogue) and
  // proj; then the LM head with its argmax candidates and the reduction that
  // also advances the device position. The embedding lookup and per-layer
  // stage 1 read the token the previous step sampled (argmaxResult), the
  // attention reads the device position: the step is captured once
  // (captureFusedStep) and replayed token after token. Its results equal the
  // key-by-key pass within the matvec tolerance (rel-L2 1e-3).
  prepareFusedStep() {
    if (this.fused) return this.fused;
    const C = this.config;
    const g = this.g;
    const c = this.ctx;
    const G = this.globals;
    const rows = this.maxSeqLen;
    let maxI = 0;
    for (let il = 0; il < C.num_layers; il++) maxI = Math.max(maxI, intermediateSize(C, il));
    const params = [];
    let ws = 0;
    for (let il = 0; il < C.num_layers; il++) {
      const swa = isSwaLayer(C, il);
      const p = { num_q_heads: C.num_q_heads, num_kv_heads: C.num_kv_heads, head_dim: headDim(C, il),
        max_seq_len: rows, scale: 1.0, sliding_window: swa ? C.sliding_window : 0, eps: C.rms_norm_eps,
        theta: ropeTheta(C, il), apply_divisor: swa ? 0 : 1 };
      params.push(p);
      ws = Math.max(ws, g.attnFusedWorkspaceSize(p));
    }
    const workspace = this.alloc(ws);
    g.memset(c, workspace, 0, ws);  // the arrival counters start (and stay) zero
    const rope = {};
    for (const glob of [false, true]) {
      const hd = glob ? C.head_dim_global : C.head_dim_local;
      const t = this.alloc(4 * rows * hd);
      g.ropeTable(c, glob ? C.rope_theta_global : C.rope_theta_swa, glob ? 1 : 0, G.rope_freqs, hd, rows, t);
      rope[glob] = t;
    }
    // the gate/up and down weights each attention launch reads into the L2
    // caches on the CUs it leaves idle (block formats only)
    const warm = [];
    for (let il = 0; il < C.num_layers; il++) {
      const L = this.layers[il];
      const F = this.formats[il] || DEFAULT_FORMATS;
      const I = intermediateSize(C, il);
      const H = C.hidden_size;
      const r = [];
      if (F.ffn_gate === 'q4k' && F.ffn_up === 'q4k') {
        r.push(g.matmulWarmRegion(c, 'q4k', I, H, L.ffn_gate), g.matmulWarmRegion(c, 'q4k', I, H, L.ffn_up));
      }
      if (F.ffn_down !== 'f16') r.push(g.matmulWarmRegion(c, F.ffn_down, H, I, L.ffn_down));
      warm.push(r);
    }
    const bytes = g.digitsBytes(maxI);
    this.fused = { params: params, workspace: workspace, workspaceBytes: ws, rope: rope, warm: warm,
      actDigits: this.alloc(bytes), pleResidual: this.alloc(4 * C.hidden_size) };
    g.sync(c);
    return this.fused;
  }

  _mv(fmt, x, w, y, M, N) {
    if (fmt === 'f16') this.g.matmulF16(this.ctx, x, w, y, { M: M, N: N, batch: 1 });
    else this.g.matmulQuant(this.ctx, x, w, y, { M: M, N: N }, fmt);
  }

  // one q/k/v launch per weight format, in order of first appearance; a
  // later one recomputes the norm and writes no residual
  _qkvGroups(groups, il, pro, H, eps) {
    const g = this.g;
    const c = this.ctx;
    const W = this.workBuffers;
    groups.forEach((grp, gi) => {
      const hOut = gi > 0 || il === 0 ? null : W.hidden;
      if (grp.fmt === 'f16') {
        g.batchPrepScale(c, Object.assign({ hOut: hOut, out: W.normed }, pro), { nparts: 1, N: H, batch: 1 }, eps);
        grp.w.forEach((w, k) => g.matmulF16(c, W.normed, w, grp.y[k], { M: grp.r[k], N: H, batch: 1 }));
      } else {
        g.normAddScaleMatmulSegments(c, grp.fmt, Object.assign({ hOut: hOut }, pro), grp.w, grp.y, grp.r, H, eps);
      }
    });
  }

  encodeFusedStep() {
    const C = this.config;
    const g = this.g;
    const c = this.ctx;
    const W = this.workBuffers;
    const G = this.globals;
    const Fz = this.prepareFusedStep();
    const H = C.hidden_size;
    const V = C.vocab_size;
    const D = C.per_layer_input_dim;
    const eps = C.rms_norm_eps;
    g.embeddingLookup(c, G.tokenEmbed, V, W.hidden, { hidden_size: H, token_id: 0 }, W.argmaxResult);
    if (D > 0) {
      g.matmulF16(c, W.hidden, G.perLayerModelProj, W.plePmProjected, { M: C.num_layers * D, N: H, batch: 1 });
      g.pleStage1Fuse(c, W.plePmProjected, G.perLayerProjNorm, G.perLayerTable, V, W.pleInputs,
        { num_layers: C.num_layers, per_layer_dim: D, eps: eps, token_id: 0 }, W.argmaxResult);
    }
    for (let il = 0; il < C.num_layers; il++) {
      const L = this.layers[il];
      const F = this.formats[il] || DEFAULT_FORMATS;
      const HD = headDim(C, il);
      const Q = C.num_q_heads * HD;
      const KV = C.num_kv_heads * HD;
      const I = intermediateSize(C, il);
      const prod = isKvProducer(C, il);
      const kv = this.kvCaches[C.kv_producer_for_layer[il]];
      // the prologue that forms this layer's normalised input
      let pro;
      if (il === 0) {
        pro = { x: W.hidden, w1: L.attn_norm, residual: null, scale: null, w2: null };
      } else {
        const P = this.layers[il - 1];
        pro = D > 0 ? { x: W.pleProjOut, w1: P.post_norm, residual: Fz.pleResidual, scale: P.layer_output_scale,
          w2: L.attn_norm } : { x: W.ffnDown, w1: P.post_ffw_norm, residual: W.residual, scale: null,
          w2: L.attn_norm };
      }
      // q/k/v grouped by weight format, in order of first appearance
      const mats = prod ? [['attn_q', W.q, Q], ['attn_k', W.k, KV], ['attn_v', W.v, KV]] : [['attn_q', W.q, Q]];
      const groups = [];
      for (const [name, y, r] of mats) {
        let grp = groups.find((x) => x.fmt === F[name]);
        if (!grp) {
          grp = { fmt: F[name], w: [], y: [], r: [] };
          groups.push(grp);
        }
        grp.w.push(L[name]);
        grp.y.push(y);
        grp.r.push(r);
      }
      const attnBufs = { qNorm: L.attn_q_norm, kNorm: prod ? L.attn_k_norm : null, ropeFreqs: G.rope_freqs,
        kCache: kv.k, vCache: kv.v, out: W.attnOut, workspace: Fz.workspace, position: W.position,
        ropeCs: Fz.rope[!isSwaLayer(C, il)] };
      if (groups.length === 1 && groups[0].fmt === 'q4k') {
        // q/k/v and the attention block: one launch where the shape allows
        g.qkvAttnDecodeFused(c, Object.assign({ hOut: il === 0 ? null : W.hidden }, pro), groups[0].w, groups[0].y,
          H, eps, attnBufs, Fz.params[il], Fz.workspaceBytes, this.maxSeqLen, Fz.warm[il]);
      } else {
        this._qkvGroups(groups, il, pro, H, eps);
        g.attnDecodeFused(c, Object.assign({ q: W.q, k: prod ? W.k : null, v: prod ? W.v : null }, attnBufs),
          Fz.params[il], Fz.workspaceBytes, this.maxSeqLen, Fz.warm[il]);
      }
      this._mv(F.attn_output, W.attnOut, L.attn_output, W.attnProj, H, Q);
      const pair = F.ffn_gate === 'q4k' && F.ffn_up === 'q4k';
      if (pair) {
        g.normAddGateUpGeluDigits(c, { o: W.attnProj, wPost: L.post_attention_norm, residual: W.hidden,
          wPre: L.ffn_norm, wGate: L.ffn_gate, wUp: L.ffn_up, hOut: W.residual, out: W.ffnMul, digits: Fz.actDigits },
        { M: I, N: H }, eps);
      } else {
        g.batchPrepScale(c, { x: W.attnProj, w1: L.post_attention_norm, residual: W.hidden, w2: L.ffn_norm,
          hOut: W.residual, out: W.normed }, { nparts: 1, N: H, batch: 1 }, eps);
        this._mv(F.ffn_gate, W.normed, L.ffn_gate, W.ffnGate, I, H);
        this._mv(F.ffn_up, W.normed, L.ffn_up, W.ffnUp, I, H);
        g.geluMul(c, W.ffnGate, W.ffnUp, W.ffnMul, I);
      }
      if (pair && F.ffn_down === 'q6k') g.matmulQuantDigits(c, Fz.actDigits, L.ffn_down, W.ffnDown, { M: H, N: I });
      else this._mv(F.ffn_down, W.ffnMul, L.ffn_down, W.ffnDown, H, I);
      if (D > 0) {
        g.pleGate(c, { x: W.ffnDown, w1: L.post_ffw_norm, residual: W.residual, hOut: Fz.pleResidual,
          wGate: L.inp_gate, pleInputs: W.pleInputs, out: W.pleGated },
        { M: D, N: H, ple_stride: 0, layer_offset: il * D, batch: 1 }, eps);
        g.matmulF16(c, W.pleGated, L.proj, W.pleProjOut, { M: H, N: D, batch: 1 });
      }
    }
    const last = this.layers[C.num_layers - 1];
    let head;
    if (D > 0) {  // the last per-layer-embedding tail, then the head normalises it
      g.batchPrepScale(c, { x: W.pleProjOut, w1: last.post_norm, residual: Fz.pleResidual,
        scale: last.layer_output_scale, hOut: W.hidden, out: W.normed }, { nparts: 1, N: H, batch: 1 }, eps);
      head = { x: W.hidden, w1: G.finalNorm, residual: null, w2: null, hOut: null };
    } else {
      head = { x: W.ffnDown, w1: last.post_ffw_norm, residual: W.residual, w2: G.finalNorm, hOut: W.hidden };
    }
    const fmt = G.lmHeadFormat || 'q6k';
    const cap = C.final_logit_softcapping;
    if (fmt === 'f16') {
      g.batchPrepScale(c, Object.assign({ out: W.normed }, head), { nparts: 1, N: H, batch: 1 }, eps);
      g.matmulF16(c, W.normed, G.lmHead, W.logits, { M: V, N: H, batch: 1 });
      if (cap > 0) g.logitSoftcap(c, W.logits, { size: V, cap: cap });
      g.argmaxAdvance(c, W.logits, W.argmaxResult, V, W.position, 1);
    } else {
      g.normAddMatmulArgmax(c, fmt, Object.assign({ weight: G.lmHead, logits: W.logits, result: W.argmaxResult,
        positions: W.position }, head), V, H, eps, cap, 1);
    }
  }

  // The fused step captured as a graph (replay with g.graphLaunch; destroy
  // with g.graphDestroy).
  captureFusedStep() {
    this.prepareFusedStep();
    this.g.graphBegin(this.ctx);
    try {
      this.encodeFusedStep();
    } catch (e) {
      this.g.graphEnd(this.ctx);
      throw e;
    }
    return this.g.graphEnd(this.ctx);
  }

  setToken(token) {
    this.g.upload(this.ctx, this.workBuffers.argmaxResult, new Uint32Array([token]));
  }

  // One greedy forward: returns nothing; readToken() reads the sample.
  forward(tokenId, position) {
    this.encodeTransformerPass(tokenId, position, false);
    this.sampleNextToken(true, false);
  }

  setPosition(position) {
    this.g.upload(this.ctx, this.workBuffers.position, new Uint32Array([position]));
  }

  readToken() {
    return this.g.download(this.ctx, this.workBuffers.argmaxResult, 4).readUInt32LE(0);
  }

  // The sampled token as a Promise: the copy is enqueued behind the work
  // already submitted and completes off the event loop (mapAsync,
  // src/engine.ts:1772-1787).
  readTokenAsync() {
    return this.g.downloadAsync(this.ctx, this.workBuffers.argmaxResult, 4).then((b) => b.readUInt32LE(0));
  }

  // Greedy generation from `token` at `position` with the captured fused
  // step, pipelined as src/engine.ts:2041-2124 does: step N + 1 is submitted
  // before step N's token is awaited (depth 2 by default), each step reading
  // the previous step's token and position on the device. Stops after
  // maxTokens, at the last position the cache holds, or at a token in
  // opts.stopTokens, which is not returned (isHardStop, :2092-2101; a step
  // already in flight behind it completes and its token is dropped).
  // Resolves to the generated tokens in order.
  async generate(token, position, maxTokens, opts) {
    const o = opts || {};
    const depth = Math.max(1, o.depth || 2);
    const stop = new Set(o.stopTokens || []);
    const steps = Math.max(0, Math.min(maxTokens, this.maxSeqLen - 1 - position));
    if (!this.fusedGraph) this.fusedGraph = this.captureFusedStep();
    this.setToken(token);
    this.setPosition(position);
    const out = [];
    const inflight = [];
    let stopped = false;
    const take = (t) => {
      if (stopped) return;
      if (stop.has(t)) stopped = true;
      else out.push(t);
    };
    for (let i = 0; i < steps && !stopped; i++) {
      this.g.graphLaunch(this.ctx, this.fusedGraph);
      inflight.push(this.readTokenAsync());
      if (inflight.length >= depth) take(await inflight.shift());
    }
    while (inflight.length) take(await inflight.shift());
    return out;
  }

  // ---- batched prefill ---------------------------------------------------
  // The ragged multi-sequence step of g4hip/decoder.py (BatchDecoder.step)
  // over `rows` rows that are tokens of this backend's one sequence: the
  // paged keys over an identity page table, so that the pool of pages of 16
  // rows IS the decode step's [maxSeqLen][num_kv_heads][head_dim] cache and
  // the fused step continues from what the prefill appended.
  _prepareBatch(B) {
    if (this.batch && this.batch.B === B) return this.batch;
    this._freeBatch();
    const C = this.config;
    const g = this.g;
    const c = this.ctx;
    const H = C.hidden_size;
    const V = C.vocab_size;
    const D = C.per_layer_input_dim;
    const NL = C.num_layers;
    if (B < 1 || B > 64) throw new Error('prefill rows: 1..64');
    let maxHd = 0;
    let maxI = 0;
    for (let il = 0; il < NL; il++) {
      maxHd = Math.max(maxHd, headDim(C, il));
      maxI = Math.max(maxI, intermediateSize(C, il));
    }
    const Q = C.num_q_heads * maxHd;
    const KV = C.num_kv_heads * maxHd;
    const own = [];
    const al = (bytes) => {
      const p = g.alloc(c, bytes);
      own.push(p);
      return p;
    };
    const f4 = (n) => al(4 * n);
    const pageSize = 16;
    const pages = Math.ceil(this.maxSeqLen / pageSize);
    const ident = new Int32Array(B * pages);
    for (let r = 0; r < B; r++) for (let p = 0; p < pages; p++) ident[r * pages + p] = p;
    const F = (il) => this.formats[il] || DEFAULT_FORMATS;
    const handoff = (il) => F(il).ffn_gate === 'q4k' && F(il).ffn_up === 'q4k' && F(il).ffn_down === 'q6k' &&
      (intermediateSize(C, il) === 6144 || intermediateSize(C, il) === 12288);
    let anyHandoff = false;
    let anyUnpaired = false;
    for (let il = 0; il < NL; il++) {
      anyHandoff = anyHandoff || handoff(il);
      anyUnpaired = anyUnpaired || !(F(il).ffn_gate === 'q4k' && F(il).ffn_up === 'q4k');
    }
    const b = { B: B, own: own, pageSize: pageSize, pages: pages, handoff: handoff,
      pageTable: al(4 * B * pages), seqLens: al(4 * B), tokens: al(4 * B),
      hidden: f4(B * H), hidden2: f4(B * H), xn: f4(B * H), xops: al(g.batchOperandBytes(H, B)),
      ksH: H / 256, ksQ: Q / 256, ksF: maxI / 256,
      q: f4(B * Q), attn: f4(B * Q), act: f4(B * maxI), logits: f4(B * V) };
    g.upload(c, b.pageTable, ident);
    Object.assign(b, { qParts: f4(b.ksH * B * Q), kParts: f4(b.ksH * B * KV), vParts: f4(b.ksH * B * KV),
      oParts: f4(b.ksQ * B * H), downParts: f4(b.ksF * B * H) });
    // the attention output also as the o projection's operand blocks (heads
    // of whole super-blocks)
    b.aops = C.head_dim_local % 256 === 0 ? al(g.batchOperandBytes(Q, B)) : null;
    b.dops = anyHandoff ? al(g.batchSubOperandBytes(maxI, B)) : null;
    if (anyUnpaired) Object.assign(b, { gate: f4(B * maxI), up: f4(B * maxI) });
    if (D > 0) {
      Object.assign(b, { pleProjected: f4(B * NL * D), pleInputs: f4(B * NL * D), pleGated: f4(B * D),
        pleOut: f4(B * H), hidden3: f4(B * H) });
    }
    b.pro = [];
    b.attnParams = [];
    let ws = 0;
    for (let il = 0; il < NL; il++) {
      const swa = isSwaLayer(C, il);
      const p = { num_seqs: B, num_q_heads: C.num_q_heads, num_kv_heads: C.num_kv_heads, head_dim: headDim(C, il),
        page_size: pageSize, max_pages: pages, max_seq_len: this.maxSeqLen, num_pages: pages, scale: 1.0,
        sliding_window: swa ? C.sliding_window : 0 };
      b.attnParams.push(p);
      b.pro.push(Object.assign({ eps: C.rms_norm_eps, theta: ropeTheta(C, il), apply_divisor: swa ? 0 : 1 }, p));
      ws = Math.max(ws, g.pagedAttnWorkspaceSize(p));
    }
    b.workspace = al(ws);
    b.workspaceBytes = ws;
    g.memset(c, b.workspace, 0, ws);
    g.sync(c);
    this.batch = b;
    return b;
  }

  _freeBatch() {
    if (!this.batch) return;
    for (const p of this.batch.own) this.g.free(this.ctx, p);
    this.batch = null;
  }

  // y = W . x for the batch rows: f16 rows through the f16 matvec (one
  // chunk), block formats split-K into at most maxKsplit chunks; returns the
  // chunk count
  _mmBatch(fmt, x, ops, w, y, M, N, maxKsplit) {
    const b = this.batch;
    if (fmt === 'f16') {
      this.g.matmulF16(this.ctx, x, w, y, { M: M, N: N, batch: b.B });
      return 1;
    }
    return this.g.matmulSegmentsBatchPartial(this.ctx, fmt, { x: x, ops: ops }, [w], [y], [M],
      { N: N, batch: b.B, max_ksplit: maxKsplit });
  }

  // One chunk: every row embeds its token (tokens) and appends its K/V row
  // at position seqLens - 1 after the advance, then attends to the positions
  // up to it (the prologue launch appends every row before the attention
  // launch reads them). head: the final norm, LM head, softcap and argmax
  // per row.
  _encodeBatchStep(head) {
    const C = this.config;
    const g = this.g;
    const c = this.ctx;
    const G = this.globals;
    const Fz = this.prepareFusedStep();
    const b = this.batch;
    const B = b.B;
    const H = C.hidden_size;
    const V = C.vocab_size;
    const D = C.per_layer_input_dim;
    const NL = C.num_layers;
    const eps = C.rms_norm_eps;
    const dims = { nparts: 1, N: H, batch: B };
    g.embeddingLookupBatch(c, G.tokenEmbed, V, b.hidden, { hidden_size: H }, b.tokens, B);
    if (D > 0) {
      g.matmulF16(c, b.hidden, G.perLayerModelProj, b.pleProjected, { M: NL * D, N: H, batch: B });
      g.pleStage1Fuse(c, b.pleProjected, G.perLayerProjNorm, G.perLayerTable, V, b.pleInputs,
        { num_layers: NL, per_layer_dim: D, eps: eps, token_id: 0 }, b.tokens, B);
    }
    g.advanceSeqLens(c, b.seqLens, B, 1);
    let nd = 0;
    for (let il = 0; il < NL; il++) {
      const L = this.layers[il];
      const F = this.formats[il] || DEFAULT_FORMATS;
      const HD = headDim(C, il);
      const Q = C.num_q_heads * HD;
      const KV = C.num_kv_heads * HD;
      const I = intermediateSize(C, il);
      const prod = isKvProducer(C, il);
      const kv = this.kvCaches[C.kv_producer_for_layer[il]];
      if (il === 0) {
        g.batchPrep(c, { x: b.hidden, w1: L.attn_norm, out: b.xn, ops: b.xops }, dims, eps);
      } else if (D > 0) {  // the previous layer's per-layer-embedding tail
        const P = this.layers[il - 1];
        g.batchPrepScale(c, { x: b.pleOut, w1: P.post_norm, residual: b.hidden3, scale: P.layer_output_scale,
          w2: L.attn_norm, hOut: b.hidden, out: b.xn, ops: b.xops }, dims, eps);
      } else {
        const P = this.layers[il - 1];
        g.batchPrep(c, { x: b.downParts, w1: P.post_ffw_norm, residual: b.hidden2, w2: L.attn_norm, hOut: b.hidden,
          out: b.xn, ops: b.xops }, { nparts: nd, N: H, batch: B }, eps);
      }
      // q/k/v grouped by weight format (a consumer layer projects q only); f16
      // rows write whole sums, so the block formats then split K once too
      const mats = prod ? [['attn_q', b.qParts, Q], ['attn_k', b.kParts, KV], ['attn_v', b.vParts, KV]]
        : [['attn_q', b.qParts, Q]];
      const groups = [];
      for (const [name, y, r] of mats) {
        let grp = groups.find((x) => x.fmt === F[name]);
        if (!grp) {
          grp = { fmt: F[name], w: [], y: [], r: [] };
          groups.push(grp);
        }
        grp.w.push(L[name]);
        grp.y.push(y);
        grp.r.push(r);
      }
      let nq = groups.some((x) => x.fmt === 'f16') ? 1 : 0;
      for (const grp of groups) {
        if (grp.fmt === 'f16') {
          grp.w.forEach((w, k) => g.matmulF16(c, b.xn, w, grp.y[k], { M: grp.r[k], N: H, batch: B }));
          continue;
        }
        const k = g.matmulSegmentsBatchPartial(c, grp.fmt, { x: b.xn, ops: b.xops }, grp.w, grp.y, grp.r,
          { N: H, batch: B, max_ksplit: nq || b.ksH });
        if (nq && k !== nq) throw new Error('layer ' + il + ': q/k/v launches split K ' + nq + ' and ' + k + ' ways');
        nq = k;
      }
      g.pagedAttnPrologue(c, { qParts: b.qParts, kParts: prod ? b.kParts : null, vParts: prod ? b.vParts : null,
        qNorm: L.attn_q_norm, kNorm: prod ? L.attn_k_norm : null, ropeFreqs: G.rope_freqs, qOut: b.q,
        kPool: prod ? kv.k : null, vPool: prod ? kv.v : null, pageTable: b.pageTable, seqLens: b.seqLens,
        ropeCs: Fz.rope[!isSwaLayer(C, il)] }, nq, b.pro[il], this.maxSeqLen);
      const ops = HD % 256 === 0 ? b.aops : null;
      g.pagedAttnDecode(c, { q: b.q, kPool: kv.k, vPool: kv.v, pageTable: b.pageTable, seqLens: b.seqLens,
        out: b.attn, workspace: b.workspace, ops: ops }, b.attnParams[il], b.workspaceBytes);
      const no = this._mmBatch(F.attn_output, b.attn, ops, L.attn_output, b.oParts, H, Q, b.ksQ);
      g.batchPrep(c, { x: b.oParts, w1: L.post_attention_norm, residual: b.hidden, w2: L.ffn_norm, hOut: b.hidden2,
        out: b.xn, ops: b.xops }, { nparts: no, N: H, batch: B }, eps);
      if (b.handoff(il)) {
        // the product goes to the down projection as operand blocks only; K
        // in chunks of 3 super-blocks
        g.gateUpGeluBatch(c, { x: b.xn, ops: b.xops, wGate: L.ffn_gate, wUp: L.ffn_up, out: null,
          downOps: b.dops }, { M: I, N: H }, B);
        nd = g.matmulSubBatchPartial(c, b.dops, L.ffn_down, b.downParts, { M: H, K: I, batch: B,
          max_ksplit: I / 768 });
      } else {
        if (F.ffn_gate === 'q4k' && F.ffn_up === 'q4k') {
          g.gateUpGeluBatch(c, { x: b.xn, ops: b.xops, wGate: L.ffn_gate, wUp: L.ffn_up, out: b.act },
            { M: I, N: H }, B);
        } else {  // gate and up apart (whole sums), then the GELU product
          this._mmBatch(F.ffn_gate, b.xn, b.xops, L.ffn_gate, b.gate, I, H, 1);
          this._mmBatch(F.ffn_up, b.xn, b.xops, L.ffn_up, b.up, I, H, 1);
          g.geluMul(c, b.gate, b.up, b.act, B * I);
        }
        nd = this._mmBatch(F.ffn_down, b.act, null, L.ffn_down, b.downParts, H, I, b.ksF);
      }
      if (D > 0) {
        // post-FFN norm-add (h, no second norm) -> inp_gate -> gelu * ple_inputs -> proj
        g.batchPrepScale(c, { x: b.downParts, w1: L.post_ffw_norm, residual: b.hidden2, out: b.hidden3 },
          { nparts: nd, N: H, batch: B }, eps);
        g.pleGate(c, { x: b.hidden3, wGate: L.inp_gate, pleInputs: b.pleInputs, out: b.pleGated },
          { M: D, N: H, ple_stride: NL * D, layer_offset: il * D, batch: B }, eps);
        g.matmulF16(c, b.pleGated, L.proj, b.pleOut, { M: H, N: D, batch: B });
      }
    }
    if (!head) return;
    const last = this.layers[NL - 1];
    if (D > 0) {
      g.batchPrepScale(c, { x: b.pleOut, w1: last.post_norm, residual: b.hidden3, scale: last.layer_output_scale,
        w2: G.finalNorm, hOut: b.hidden, out: b.xn, ops: b.xops }, dims, eps);
    } else {
      g.batchPrep(c, { x: b.downParts, w1: last.post_ffw_norm, residual: b.hidden2, w2: G.finalNorm,
        hOut: b.hidden, out: b.xn, ops: b.xops }, { nparts: nd, N: H, batch: B }, eps);
    }
    const fmt = G.lmHeadFormat || 'q6k';
    const cap = C.final_logit_softcapping;
    if (fmt === 'f16') {
      g.matmulF16(c, b.xn, G.lmHead, b.logits, { M: V, N: H, batch: B });
      if (cap > 0) g.logitSoftcap(c, b.logits, { size: B * V, cap: cap });
    } else {
      g.matmulSegmentsBatchPartial(c, fmt, { x: b.xn, ops: b.xops }, [G.lmHead], [b.logits], [V],
        { N: H, batch: B, max_ksplit: 1 }, cap > 0 ? cap : 0);
    }
    g.argmaxBatch(c, b.logits, b.tokens, V, B);
  }

  // The prompt `tokens` at positions start, start + 1, ... through the
  // batched step, opts.rows (default 64) tokens per chunk. The reference
  // runs one forward per prompt token (src/engine.ts:1923-1938) and the LM
  // head once after the last (getFirstTokenAfterPrefill, :1951-1959); here
  // each chunk is one ragged step whose row r is token start + 64k + r, and
  // only the last chunk runs the LM head. A short last chunk repeats its
  // last token and position in the spare rows (identical rows, identical
  // writes). Leaves the greedy sample of the last token where the fused
  // step reads its token and start + T in the position counter, so
  // generate(sample, start + T, ...) continues; returns that sample.
  prefill(tokens, start, opts) {
    const o = opts || {};
    const T = tokens.length;
    const pos0 = start || 0;
    if (T === 0 || pos0 + T > this.maxSeqLen - 1) {
      throw new Error('prefill: ' + T + ' tokens from ' + pos0 + ' do not fit ' + this.maxSeqLen + ' positions');
    }
    const B = Math.min(o.rows || 64, T);
    const b = this._prepareBatch(B);
    const g = this.g;
    const c = this.ctx;
    const nch = Math.ceil(T / B);
    // every chunk's tokens and lengths before the step's advance, uploaded once
    const tok = new Uint32Array(nch * B);
    const len = new Uint32Array(nch * B);
    for (let i = 0; i < nch * B; i++) {
      const t = Math.min(i, T - 1);
      tok[i] = tokens[t];
      len[i] = pos0 + t;
    }
    const dtok = g.alloc(c, 4 * nch * B);
    const dlen = g.alloc(c, 4 * nch * B);
    try {
      g.upload(c, dtok, tok);
      g.upload(c, dlen, len);
      for (let k = 0; k < nch; k++) {
        g.copy(c, b.tokens, dtok + BigInt(4 * B * k), 4 * B);
        g.copy(c, b.seqLens, dlen + BigInt(4 * B * k), 4 * B);
        this._encodeBatchStep(k === nch - 1);
      }
      // the prompt's last token is row (T - 1) - (nch - 1) B of the last chunk
      const last = T - 1 - (nch - 1) * B;
      g.copy(c, this.workBuffers.argmaxResult, b.tokens + BigInt(4 * last), 4);
      this.setPosition(pos0 + T);
      g.sync(c);
    } finally {
      g.free(c, dtok);
      g.free(c, dlen);
    }
    return this.readToken();
  }

  readF32(name, count) {
    const b = this.g.download(this.ctx, this.workBuffers[name], 4 * count);
    return new Float32Array(b.buffer, b.byteOffset, count);
  }
}

module.exports = {
  HipBackend: HipBackend,
  loadAddon: loadAddon,
  e2bConfig: e2bConfig,
  configFromGGUF: configFromGGUF,
  kvProducerMap: kvProducerMap,
  headDim: headDim,
  intermediateSize: intermediateSize,
  isKvProducer: isKvProducer,
  LAYER_TENSORS: LAYER_TENSORS,
  PLE_TENSORS: PLE_TENSORS,
  DEFAULT_FORMATS: DEFAULT_FORMATS,
};
