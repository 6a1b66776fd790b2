'use strict';
// CPU checks of the Node host side (no GPU needed): the N-API addon loads,
// exports every key, maps library failures to JS Errors carrying the status
// name and g4_last_error(); HipBackend issues the reference's pass order
// (src/engine.ts:1505-1625 encodeTransformerPass, :1686-1746 the greedy
// sample) with each layer's shapes, and the E2B KV producer map
// (src/config/gemma4-e2b.ts:159-180). Exits non-zero on the first failure.
const assert = require('assert');
const path = require('path');

const root = path.resolve(__dirname, '..', '..');
const hb = require(path.join(root, 'gemma4-webgpu_amd', 'node', 'hip_backend.js'));

function check(name, fn) {
  fn();
  console.log('ok ' + name);
}

const KEYS = ['version', 'lastError', 'init', 'destroy', 'deviceInfo', 'alloc', 'free', 'memset', 'upload',
  'download', 'downloadAsync', 'eventRecord', 'eventQuery', 'eventWait', 'eventDestroy', 'sync', 'graphBegin', 'graphEnd', 'graphLaunch', 'graphDestroy', 'fill', 'matmulQuant',
  'matmulQuantMR4', 'kvCacheStore', 'attnScore', 'softmax', 'attnOutput', 'attnDecodeWorkspaceSize', 'attnDecode',
  'perHeadRmsNormNoWeight', 'fusedPerHeadNormRope', 'rmsNorm', 'fusedNormAdd', 'geluMul', 'logitSoftcap',
  'embeddingLookup', 'argmax', 'topk256', 'advancePosition', 'pleStage1Fuse', 'pleGeluMul', 'pleSkipScaleAdd',
  'ggufOpen', 'ggufClose', 'ggufInfo', 'ggufMetadata', 'ggufTensors', 'ggufUpload', 'ggufUploadF16', 'dequantF16',
  'digitsBytes', 'attnFusedWorkspaceSize', 'ropeTable', 'matmulWarmRegion', 'attnDecodeFused',
  'normAddScaleMatmulSegments', 'qkvAttnDecodeFused',
  'normAddGateUpGeluDigits', 'matmulQuantDigits', 'normAddMatmulArgmax', 'pleGate', 'matmulF16', 'batchPrepScale',
  'argmaxAdvance', 'batchOperandBytes', 'batchSubOperandBytes', 'pagedAttnWorkspaceSize', 'copy',
  'embeddingLookupBatch', 'advanceSeqLens', 'batchPrep', 'matmulSegmentsBatchPartial', 'pagedAttnPrologue',
  'pagedAttnDecode', 'gateUpGeluBatch', 'matmulSubBatchPartial', 'argmaxBatch', 'topk256Batch'];

const addon = hb.loadAddon();

check('addon exports every key', () => {
  assert.deepStrictEqual(Object.keys(addon).sort(), KEYS.slice().sort());
  assert.strictEqual(addon.version(), 1);
});

check('init: a context, or without a device G4_ERR_NO_DEVICE with the library message', () => {
  let err = null;
  try {
    const ctx = addon.init(0);
    assert.strictEqual(typeof ctx, 'bigint');  // a machine with a GPU
    assert.ok(addon.deviceInfo(ctx).numCus > 0);
    addon.destroy(ctx);
    return;
  } catch (e) {
    err = e;
  }
  assert.ok(err instanceof Error);
  assert.strictEqual(err.code, 'G4_ERR_NO_DEVICE');
  assert.ok(err.message.length > 0);
  assert.strictEqual(err.message, addon.lastError());
});

check('null context: a key throws G4_ERR_INVALID', () => {
  assert.throws(() => addon.rmsNorm(null, null, null, null, { hidden_size: 1536, eps: 1e-6 }),
    (e) => e.code === 'G4_ERR_INVALID' && /null context/.test(e.message));
});

check('argument types are checked before any call', () => {
  assert.throws(() => addon.rmsNorm(1, null, null, null, { hidden_size: 1536, eps: 1e-6 }),
    (e) => e instanceof TypeError && e.code === 'G4_ERR_ARG');
  assert.throws(() => addon.rmsNorm(null, null, null, null, { hidden_size: 1536 }),
    (e) => e instanceof TypeError && /eps/.test(e.message));
  assert.throws(() => addon.matmulQuant(null, null, null, null, { M: 8, N: 256 }, 'q5k'),
    (e) => e instanceof TypeError);
});

check('workspace size query needs no device', () => {
  const n = addon.attnDecodeWorkspaceSize({ num_q_heads: 8, num_kv_heads: 1, head_dim: 256, seq_len: 4096,
    scale: 1.0, sliding_window: 0 });
  assert.ok(n > 0);
});

check('E2B producer map', () => {
  const C = hb.e2bConfig();
  const want = [];
  for (let i = 0; i < 35; i++) want.push(i < 15 ? i : ([19, 24, 29, 34].indexOf(i) >= 0 ? 14 : 13));
  assert.deepStrictEqual(C.kv_producer_for_layer, want);
  assert.strictEqual(hb.headDim(C, 4), 512);
  assert.strictEqual(hb.headDim(C, 5), 256);
  assert.strictEqual(hb.intermediateSize(C, 14), 6144);
  assert.strictEqual(hb.intermediateSize(C, 15), 12288);
});

// A recording stand-in for the addon: every key logs its arguments.
function mockAddon() {
  const calls = [];
  let next = 1;
  const m = { calls: calls };
  for (const k of KEYS) m[k] = function () { calls.push([k].concat(Array.prototype.slice.call(arguments))); };
  m.alloc = () => BigInt(4096 * next++);
  m.init = () => 'ctx';
  m.digitsBytes = function () {
    calls.push(['digitsBytes'].concat(Array.prototype.slice.call(arguments)));
    return 4096;
  };
  m.matmulWarmRegion = function (ctx, wtype, M, N, w) {
    calls.push(['matmulWarmRegion', ctx, wtype, M, N, w]);
    return { base: w, totalBytes: M * N, wgBytes: 1024, nwgs: 8 };
  };
  m.attnFusedWorkspaceSize = function (p) {
    calls.push(['attnFusedWorkspaceSize', p]);
    return 1024 + p.head_dim;
  };
  m.batchOperandBytes = (N, b) => N * b;
  m.batchSubOperandBytes = (K, b) => 2 * K * b;
  m.pagedAttnWorkspaceSize = (p) => 64 * p.head_dim;
  // the K split of a batched matmul: the most the caller allows, at most 6
  m.matmulSegmentsBatchPartial = function () {
    calls.push(['matmulSegmentsBatchPartial'].concat(Array.prototype.slice.call(arguments)));
    return Math.min(6, arguments[6].max_ksplit);
  };
  m.matmulSubBatchPartial = function () {
    calls.push(['matmulSubBatchPartial'].concat(Array.prototype.slice.call(arguments)));
    return arguments[4].max_ksplit;
  };
  m.download = function () {
    calls.push(['download'].concat(Array.prototype.slice.call(arguments)));
    return Buffer.alloc(arguments[2]);
  };
  return m;
}

// The reference's passes for one layer (src/engine.ts:1544-1616, the
// matmulQuantMR4 gate/up branch, PLE stage 2 at the end).
function layerPasses(producer) {
  const p = [['attn.rmsNorm', 'rmsNorm']];
  if (producer) {
    for (let i = 0; i < 3; i++) p.push(['attn.linearQKV.producer', 'matmulQuant']);
    p.push(['attn.vNorm', 'perHeadRmsNormNoWeight']);
    p.push(['attn.fusedNormRopeQK', 'fusedPerHeadNormRope'], ['attn.fusedNormRopeQK', 'fusedPerHeadNormRope']);
    p.push(['attn.kvCacheStore', 'kvCacheStore']);
  } else {
    p.push(['attn.linearQ.consumer', 'matmulQuant'], ['attn.fusedNormRopeQ', 'fusedPerHeadNormRope']);
  }
  return p.concat([['attn.attnScore', 'attnScore'], ['attn.softmax', 'softmax'], ['attn.attnOutput', 'attnOutput'],
    ['attn.linearOut', 'matmulQuant'], ['attn.postNormAdd', 'fusedNormAdd'], ['ffn.rmsNorm', 'rmsNorm'],
    ['ffn.linearGateUp', 'matmulQuantMR4'], ['ffn.linearGateUp', 'matmulQuantMR4'], ['ffn.geluMul', 'geluMul'],
    ['ffn.linearDown', 'matmulQuant'], ['ffn.postNormAdd', 'fusedNormAdd'],
    ['ple2.linearInpGate', 'matmulQuant'], ['ple2.geluMul', 'pleGeluMul'], ['ple2.linearPostProj', 'matmulQuant'],
    ['ple2.rmsNorm', 'rmsNorm'], ['ple2.skipScaleAdd', 'pleSkipScaleAdd']]);
}

const PLE_GLOBALS = { perLayerModelProj: 'pmp', perLayerProjNorm: 'ppn', perLayerTable: 'plt' };

check('HipBackend replays the reference pass order with per-layer shapes', () => {
  const C = hb.e2bConfig();
  const m = mockAddon();
  const trace = [];
  const be = new hb.HipBackend(m, 'ctx', C, { maxSeqLen: 4096, trace: trace });
  be.allocate();
  const tensors = (il) => {
    const t = {};
    for (const n of Object.keys(be.layerTensorBytes(il))) t[n] = 'L' + il + '.' + n;
    return t;
  };
  for (let il = 0; il < 35; il++) be.setLayerWeights(il, tensors(il));
  assert.throws(() => be.setGlobals({ tokenEmbed: 'emb', lmHead: 'head', finalNorm: 'fnorm', rope_freqs: 'rf' }),
    /perLayerModelProj/);
  be.setGlobals(Object.assign({ tokenEmbed: 'emb', lmHead: 'head', finalNorm: 'fnorm', rope_freqs: 'rf' },
    PLE_GLOBALS));
  m.calls.length = 0;
  const pos = 700;
  be.encodeTransformerPass(42, pos, false);
  be.sampleNextToken(true, false);
  let want = [['embed', 'embeddingLookup'], ['ple1.pmProj', 'matmulQuant'], ['ple1.stage1Fuse', 'pleStage1Fuse']];
  for (let il = 0; il < 35; il++) want = want.concat(layerPasses(il < 15));
  want = want.concat([['final.rmsNorm', 'rmsNorm'], ['lmHead', 'matmulQuant'], ['logitSoftcap', 'logitSoftcap'],
    ['sample.argmax', 'argmax']]);
  assert.deepStrictEqual(trace, want);
  assert.deepStrictEqual(m.calls.map((c) => c[0]), want.map((w) => w[1]));

  // per-layer shapes and bindings of the calls
  let at = 3;
  const W = be.workBuffers;
  assert.deepStrictEqual(m.calls[0].slice(1, 6), ['ctx', 'emb', 262144, W.hidden, { hidden_size: 1536, token_id: 42 }]);
  assert.deepStrictEqual(m.calls[1].slice(1, 7), ['ctx', W.hidden, 'pmp', W.plePmProjected, { M: 35 * 256, N: 1536 },
    'f16']);
  assert.deepStrictEqual(m.calls[2].slice(1, 9), ['ctx', W.plePmProjected, 'ppn', 'plt', 262144, W.pleInputs,
    { num_layers: 35, per_layer_dim: 256, eps: 1e-6, token_id: 42 }, null]);
  for (let il = 0; il < 35; il++) {
    const n = layerPasses(il < 15).length;
    const calls = m.calls.slice(at, at + n);
    at += n;
    const hd = [4, 9, 14, 19, 24, 29, 34].indexOf(il) >= 0 ? 512 : 256;
    const glob = hd === 512;
    const I = il < 15 ? 6144 : 12288;
    const src = C.kv_producer_for_layer[il];
    const by = (k) => calls.filter((c) => c[0] === k);
    assert.deepStrictEqual(by('matmulQuant')[0].slice(3, 6), ['L' + il + '.attn_q', W.q, { M: 8 * hd, N: 1536 }]);
    const rope = by('fusedPerHeadNormRope')[0][4];
    assert.deepStrictEqual(rope, { num_heads: 8, head_dim: hd, eps: 1e-6, position: pos, theta: glob ? 1e6 : 1e4,
      apply_divisor: glob ? 1 : 0 });
    const score = by('attnScore')[0];
    assert.strictEqual(score[3], be.kvCaches[src].k);
    assert.deepStrictEqual(score[5], { num_q_heads: 8, num_kv_heads: 1, head_dim: hd, seq_len: pos + 1, scale: 1.0,
      sliding_window: glob ? 0 : 512 });
    assert.strictEqual(by('attnOutput')[0][3], be.kvCaches[src].v);
    assert.deepStrictEqual(by('matmulQuantMR4')[0][5], { M: I, N: 1536 });
    assert.deepStrictEqual(by('matmulQuant').filter((c) => c[3] === 'L' + il + '.ffn_down')[0].slice(3, 7),
      ['L' + il + '.ffn_down', W.ffnDown, { M: 1536, N: I }, 'q6k']);
    const mqs = by('matmulQuant');
    assert.deepStrictEqual(mqs[mqs.length - 2].slice(2, 7), [W.hidden, 'L' + il + '.inp_gate', W.pleGate,
      { M: 256, N: 1536 }, 'f16']);
    assert.deepStrictEqual(mqs[mqs.length - 1].slice(2, 7), [W.pleGated, 'L' + il + '.proj', W.pleProjOut,
      { M: 1536, N: 256 }, 'f16']);
    assert.deepStrictEqual(by('pleGeluMul')[0].slice(2, 6), [W.pleGate, W.pleInputs, W.pleGated,
      { layer_offset: il * 256, size: 256 }]);
    assert.deepStrictEqual(by('pleSkipScaleAdd')[0].slice(2, 6), [W.hidden, W.plePostNormed,
      'L' + il + '.layer_output_scale', { size: 1536 }]);
    if (il < 15) {
      const st = by('kvCacheStore')[0];
      assert.deepStrictEqual(st.slice(4, 7), [be.kvCaches[il].k, be.kvCaches[il].v,
        { num_kv_heads: 1, head_dim: hd, position: pos, max_seq_len: 4096 }]);
    } else {
      assert.strictEqual(by('kvCacheStore').length, 0);
      assert.strictEqual(be.kvCaches[il], be.kvCaches[src]);
    }
  }
});

check('device-side token and position: the pass reads them, the sample advances the position', () => {
  const bad = hb.e2bConfig({ num_layers: 2, num_unshared_layers: 1, global_layers: [1], vocab_size: 4096 });
  assert.throws(() => new hb.HipBackend(mockAddon(), 'ctx', bad, {}).allocate(), /no unshared layer/);
  const C = hb.e2bConfig({ num_layers: 3, num_unshared_layers: 2, global_layers: [1], vocab_size: 4096 });
  const m = mockAddon();
  const be = new hb.HipBackend(m, 'ctx', C, { maxSeqLen: 1024 });
  be.allocate();
  for (let il = 0; il < 3; il++) {
    const t = {};
    for (const n of Object.keys(be.layerTensorBytes(il))) t[n] = n;
    be.setLayerWeights(il, t);
  }
  be.setGlobals(Object.assign({ tokenEmbed: 'emb', lmHead: 'head', finalNorm: 'fnorm', rope_freqs: 'rf' },
    PLE_GLOBALS));
  m.calls.length = 0;
  be.encodeTransformerPass(null, 0, true);
  be.sampleNextToken(true, true);
  const W = be.workBuffers;
  assert.strictEqual(m.calls[0][6], W.argmaxResult);            // embedding of the sampled token
  assert.strictEqual(m.calls[2][0], 'pleStage1Fuse');
  assert.strictEqual(m.calls[2][8], W.argmaxResult);            // and its per-layer-embedding row
  for (const c of m.calls.filter((x) => ['attnScore', 'attnOutput'].indexOf(x[0]) >= 0)) {
    assert.strictEqual(c[6], W.position);
    assert.strictEqual(c[5].seq_len, 1024);                      // the bound, the device value is read
  }
  assert.strictEqual(m.calls.filter((x) => x[0] === 'kvCacheStore')[0][7], W.position);
  const last = m.calls[m.calls.length - 1];
  assert.deepStrictEqual(last, ['advancePosition', 'ctx', W.position, 1]);
  assert.throws(() => be.setLayerWeights(0, {}), /missing tensor/);
});

check('per-tensor formats: sizes, wtypes, f16 rows, the LM head and the 4-row gate/up only for Q4_K', () => {
  const C = hb.e2bConfig({ num_layers: 2, num_unshared_layers: 2, global_layers: [1], vocab_size: 4096,
    per_layer_input_dim: 0 });
  const m = mockAddon();
  const be = new hb.HipBackend(m, 'ctx', C, { maxSeqLen: 1024 });
  be.allocate();
  const F = { attn_v: 'q6k', ffn_down: 'q4k', attn_output: 'f16' };
  const sizes = be.layerTensorBytes(0, F);
  assert.strictEqual(sizes.attn_v, 256 * 1536 / 256 * 210);
  assert.strictEqual(sizes.ffn_down, 1536 * 6144 / 256 * 144);
  assert.strictEqual(sizes.attn_output, 2 * 1536 * 2048);
  assert.strictEqual(sizes.inp_gate, undefined);
  const t = (il, f) => {
    const o = {};
    for (const n of Object.keys(be.layerTensorBytes(il, f))) o[n] = n + il;
    return o;
  };
  be.setLayerWeights(0, t(0, F), F);
  be.setLayerWeights(1, t(1, { ffn_gate: 'q6k' }), { ffn_gate: 'q6k' });
  assert.throws(() => be.setLayerWeights(1, t(1), { attn_q: 'q5k' }), /format/);
  be.setGlobals({ tokenEmbed: 'emb', lmHead: 'head', finalNorm: 'fnorm', rope_freqs: 'rf', lmHeadFormat: 'q4k' });
  m.calls.length = 0;
  be.forward(7, 3);
  const mq = m.calls.filter((c) => c[0] === 'matmulQuant' || c[0] === 'matmulQuantMR4');
  const fmt = (name) => mq.filter((c) => c[3] === name)[0];
  assert.strictEqual(fmt('attn_v0')[6], 'q6k');
  assert.strictEqual(fmt('attn_output0')[6], 'f16');
  assert.strictEqual(fmt('attn_output1')[6], 'q4k');
  assert.strictEqual(fmt('attn_k0')[6], 'q4k');
  assert.strictEqual(fmt('ffn_down0')[6], 'q4k');
  assert.strictEqual(fmt('ffn_down1')[6], 'q6k');
  assert.strictEqual(fmt('ffn_gate0')[0], 'matmulQuantMR4');
  assert.strictEqual(fmt('ffn_gate1')[0], 'matmulQuant');
  assert.strictEqual(fmt('ffn_gate1')[6], 'q6k');
  assert.strictEqual(fmt('head')[6], 'q4k');
  assert.strictEqual(m.calls.filter((c) => /^ple/.test(c[0])).length, 0);
});

check('the fused step: launch order, prologue chaining, format groups, PLE and the head', () => {
  const C = hb.e2bConfig({ num_layers: 4, num_unshared_layers: 2, global_layers: [1, 3], vocab_size: 4096 });
  const m = mockAddon();
  const be = new hb.HipBackend(m, 'ctx', C, { maxSeqLen: 1024 });
  be.allocate();
  const t = (il, f) => {
    const o = {};
    for (const n of Object.keys(be.layerTensorBytes(il, f))) o[n] = n + il;
    return o;
  };
  const F1 = { attn_v: 'q6k', ffn_gate: 'f16' };  // layer 1: two q/k/v launches, unfused FFN
  be.setLayerWeights(0, t(0), {});
  be.setLayerWeights(1, t(1, F1), F1);
  be.setLayerWeights(2, t(2), {});
  be.setLayerWeights(3, t(3), { ffn_down: 'q4k' });
  be.setGlobals(Object.assign({ tokenEmbed: 'emb', lmHead: 'head', finalNorm: 'fnorm', rope_freqs: 'rf' },
    PLE_GLOBALS));
  m.calls.length = 0;
  be.encodeFusedStep();
  const keys = m.calls.map((x) => x[0]);
  assert.strictEqual(keys.filter((k) => k === 'attnFusedWorkspaceSize').length, 4);
  assert.strictEqual(keys.filter((k) => k === 'ropeTable').length, 2);
  const step = keys.filter((k) => ['alloc', 'memset', 'sync', 'attnFusedWorkspaceSize', 'ropeTable',
    'digitsBytes', 'matmulWarmRegion'].indexOf(k) < 0);
  // layers whose q/k/v are all Q4_K issue them with the attention
  // (qkvAttnDecodeFused); layer 1 (a Q6_K v) makes two q/k/v launches and
  // the attention's own
  const tail = (ffn, down) => ['matmulQuant'].concat(ffn, [down], ['pleGate', 'matmulF16']);
  const want = ['embeddingLookup', 'matmulF16', 'pleStage1Fuse']
    .concat(['qkvAttnDecodeFused'], tail(['normAddGateUpGeluDigits'], 'matmulQuantDigits'))
    .concat(['normAddScaleMatmulSegments', 'normAddScaleMatmulSegments', 'attnDecodeFused'],
      tail(['batchPrepScale', 'matmulF16', 'matmulQuant', 'geluMul'], 'matmulQuant'))
    .concat(['qkvAttnDecodeFused'], tail(['normAddGateUpGeluDigits'], 'matmulQuantDigits'))
    .concat(['qkvAttnDecodeFused'], tail(['normAddGateUpGeluDigits'], 'matmulQuant'))
    .concat(['batchPrepScale', 'normAddMatmulArgmax']);
  assert.deepStrictEqual(step, want);
  // qkvAttnDecodeFused(ctx, pro, weights, outputs, N, eps, buffers, params, wsBytes, ropeRows, regions)
  const qa = m.calls.filter((x) => x[0] === 'qkvAttnDecodeFused');
  // layer 0 normalises the embedding and writes no residual
  assert.strictEqual(qa[0][2].x, be.workBuffers.hidden);
  assert.strictEqual(qa[0][2].hOut, null);
  assert.deepStrictEqual(qa[0][3], ['attn_q0', 'attn_k0', 'attn_v0']);
  assert.deepStrictEqual(qa[0][4], [be.workBuffers.q, be.workBuffers.k, be.workBuffers.v]);
  const nas = m.calls.filter((x) => x[0] === 'normAddScaleMatmulSegments');
  // layer 1's first launch adds the previous PLE tail and writes the
  // residual, its second (the Q6_K v) recomputes the norm and writes none
  assert.strictEqual(nas[0][3].x, be.workBuffers.pleProjOut);
  assert.strictEqual(nas[0][3].scale, 'layer_output_scale0');
  assert.strictEqual(nas[0][3].hOut, be.workBuffers.hidden);
  assert.deepStrictEqual([nas[0][2], nas[0][4]], ['q4k', ['attn_q1', 'attn_k1']]);
  assert.deepStrictEqual([nas[1][2], nas[1][4], nas[1][3].hOut], ['q6k', ['attn_v1'], null]);
  // consumer layers (2, 3) project q only and read their producer's cache
  assert.deepStrictEqual([qa[1][3], qa[1][4]], [['attn_q2'], [be.workBuffers.q]]);
  assert.strictEqual(qa[1][2].hOut, be.workBuffers.hidden);
  assert.strictEqual(qa[1][7].kNorm, null);
  assert.strictEqual(qa[1][7].kCache, be.kvCaches[0].k);
  assert.strictEqual(qa[2][7].kCache, be.kvCaches[1].k);
  const att = m.calls.filter((x) => x[0] === 'attnDecodeFused');
  assert.strictEqual(att.length, 1);
  assert.strictEqual(att[0][2].k, be.workBuffers.k);
  assert.strictEqual(att[0][3].sliding_window, 0);
  assert.strictEqual(att[0][3].head_dim, 512);
  assert.strictEqual(qa[0][8].sliding_window, 512);
  // L2 warming: layer 0 the gate/up pair and the down, layer 1 (f16 gate) the down only
  assert.deepStrictEqual(qa[0][11].map((r) => r.base), ['ffn_gate0', 'ffn_up0', 'ffn_down0']);
  assert.deepStrictEqual(att[0][6].map((r) => r.base), ['ffn_down1']);
  const head = m.calls.filter((x) => x[0] === 'normAddMatmulArgmax')[0];
  assert.strictEqual(head[2], 'q6k');
  assert.strictEqual(head[3].positions, be.workBuffers.position);
  assert.strictEqual(head[3].result, be.workBuffers.argmaxResult);
});

check('prefill: the batched step over the decode caches, LM head on the last chunk only', () => {
  const C = hb.e2bConfig();
  const m = mockAddon();
  const be = new hb.HipBackend(m, 'ctx', C, { maxSeqLen: 1000 });
  be.allocate();
  for (let il = 0; il < C.num_layers; il++) {
    const t = {};
    for (const n of Object.keys(be.layerTensorBytes(il))) t[n] = n + il;
    be.setLayerWeights(il, t);
  }
  be.setGlobals(Object.assign({ tokenEmbed: 'emb', lmHead: 'head', finalNorm: 'fn', rope_freqs: 'rf' },
    PLE_GLOBALS));
  const toks = [];
  for (let i = 0; i < 20; i++) toks.push(1000 + i);
  m.calls.length = 0;
  be.prefill(toks, 600, { rows: 8 });
  const b = be.batch;
  const of = (k) => m.calls.filter((x) => x[0] === k);
  assert.strictEqual(b.B, 8);
  assert.strictEqual(b.pages, 63);  // 1000 positions in pages of 16
  // the identity page table, one list per row
  const table = of('upload').find((x) => x[2] === b.pageTable)[3];
  assert.strictEqual(table.length, 8 * 63);
  for (let r = 0; r < 8; r++) for (let p = 0; p < 63; p++) assert.strictEqual(table[r * 63 + p], p);
  // chunk tokens and lengths: 20 tokens, the last chunk's spare rows repeat token 19 at position 619
  const up = of('upload').filter((x) => x[3] instanceof Uint32Array && x[3].length === 24);
  assert.deepStrictEqual(Array.from(up[0][3]), toks.concat([1019, 1019, 1019, 1019]));
  const lens = [];
  for (let i = 0; i < 24; i++) lens.push(600 + Math.min(i, 19));
  assert.deepStrictEqual(Array.from(up[1][3]), lens);
  const copies = of('copy');
  assert.deepStrictEqual(copies.slice(0, 6).map((x) => [x[2], x[3] - up[x[2] === b.tokens ? 0 : 1][2], x[4]]),
    [[b.tokens, 0n, 32], [b.seqLens, 0n, 32], [b.tokens, 32n, 32], [b.seqLens, 32n, 32], [b.tokens, 64n, 32],
      [b.seqLens, 64n, 32]]);
  // the first sample: row 3 of the last chunk, where the fused step reads its token
  assert.deepStrictEqual(copies[6].slice(2), [be.workBuffers.argmaxResult, b.tokens + 12n, 4]);
  assert.deepStrictEqual(Array.from(of('upload').pop()[3]), [620]);  // the position after the prompt
  assert.strictEqual(of('embeddingLookupBatch').length, 3);
  assert.strictEqual(of('advanceSeqLens').length, 3);
  assert.strictEqual(of('argmaxBatch').length, 1);
  assert.strictEqual(of('pagedAttnDecode').length, 3 * C.num_layers);
  // a consumer layer projects q only and attends over its producer's cache
  const pro = of('pagedAttnPrologue');
  const dec = of('pagedAttnDecode');
  for (let il = 0; il < C.num_layers; il++) {
    const src = C.kv_producer_for_layer[il];
    const p = pro[il][2];
    assert.strictEqual(p.kPool, il === src ? be.kvCaches[il].k : null);
    assert.strictEqual(p.kParts, il === src ? b.kParts : null);
    assert.strictEqual(dec[il][2].kPool, be.kvCaches[src].k);
    assert.strictEqual(pro[il][4].max_seq_len, 1000);
    assert.strictEqual(pro[il][4].num_pages, 63);
    assert.strictEqual(pro[il][4].head_dim, hb.headDim(C, il));
    assert.strictEqual(pro[il][3], 6);  // the q/k/v launch's K split
  }
  // Q4_K gate/up over a Q6_K down: the product handed over as operand blocks
  const gu = of('gateUpGeluBatch');
  assert.strictEqual(gu.length, 3 * C.num_layers);
  assert.ok(gu.every((x) => x[2].downOps === b.dops && x[2].out === null));
  assert.strictEqual(of('matmulSubBatchPartial')[0][5].max_ksplit, 8);  // 6144 / 768
  be.close();
  assert.strictEqual(be.batch, null);
});

console.log('all node CPU checks passed');

// generate(): step N + 1 is submitted before step N's token is awaited
// (src/engine.ts:2041-2124 depth 2); each readback resolves on a later turn
// of the event loop, as a real one completes off the loop.
async function checkPipelinedGenerate() {
  const C = hb.e2bConfig();
  const m = mockAddon();
  const be = new hb.HipBackend(m, 'ctx', C, { maxSeqLen: 4096 });
  be.allocate();
  be.fusedGraph = 'graph';  // (capture is checked by the fused-step checks)
  const log = [];
  let n = 0;
  m.graphLaunch = (ctx, g) => {
    assert.strictEqual(g, 'graph');
    log.push('launch');
  };
  const tokenAt = (i) => (i === 2 ? 1 : 100 + i);
  m.downloadAsync = (ctx, src, bytes) => {
    assert.strictEqual(src, be.workBuffers.argmaxResult);
    assert.strictEqual(bytes, 4);
    const i = n++;
    log.push('read' + i);
    return new Promise((resolve) => setImmediate(() => {
      log.push('done' + i);
      const b = Buffer.alloc(4);
      b.writeUInt32LE(tokenAt(i), 0);
      resolve(b);
    }));
  };
  let toks = await be.generate(7, 600, 4);
  assert.deepStrictEqual(toks, [100, 101, 1, 103]);
  assert.deepStrictEqual(log, ['launch', 'read0', 'launch', 'read1', 'done0', 'launch', 'read2', 'done1', 'launch',
    'read3', 'done2', 'done3']);
  const uploads = m.calls.filter((c) => c[0] === 'upload');
  assert.deepStrictEqual(Array.from(uploads[uploads.length - 2][3]), [7]);    // the first token
  assert.deepStrictEqual(Array.from(uploads[uploads.length - 1][3]), [600]);  // its position
  console.log('ok generate pipelines depth 2');
  // a stop token: not returned; the step in flight behind it completes, its token is dropped
  log.length = 0;
  n = 0;
  toks = await be.generate(7, 600, 10, { stopTokens: [1] });
  assert.deepStrictEqual(toks, [100, 101]);
  assert.deepStrictEqual(log, ['launch', 'read0', 'launch', 'read1', 'done0', 'launch', 'read2', 'done1', 'launch',
    'read3', 'done2', 'done3']);
  console.log('ok generate stops at a stop token');
  // depth 1: each token is awaited before the next step is submitted
  log.length = 0;
  n = 0;
  toks = await be.generate(7, 600, 2, { depth: 1 });
  assert.deepStrictEqual(toks, [100, 101]);
  assert.deepStrictEqual(log, ['launch', 'read0', 'done0', 'launch', 'read1', 'done1']);
  console.log('ok generate depth 1');
  // no step past the cache's last position
  log.length = 0;
  n = 0;
  toks = await be.generate(7, 4093, 10);
  assert.deepStrictEqual(toks, [100, 101]);
  assert.strictEqual(log.filter((e) => e === 'launch').length, 2);
  console.log('ok generate stops at the cache capacity');
}

checkPipelinedGenerate().catch((e) => {
  console.error(e);
  process.exit(1);
});
