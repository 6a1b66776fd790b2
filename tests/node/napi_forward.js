'use strict';
// GPU run of HipBackend through the N-API addon (driven by
// tests/test_gpu_napi.py, which writes the model and checks the outputs
// against the oracle): usage `node napi_forward.js <dir>`.
//   <dir>/config.json  {overrides (e2bConfig), maxSeqLen, position, token,
//                       formats (per layer: {matrix: 'q4k' | 'q6k'})}, or
//                      {gguf (a model file: HipBackend.fromGGUF, zero
//                       caches), maxSeqLen, position, token}
//   <dir>/<name>.bin   raw tensor bytes: L<il>.<tensor> per layer, kv<il>.k /
//                      kv<il>.v (initial f16 caches of the producer layers),
//                      tokenEmbed, lmHead, finalNorm, rope_freqs, and with
//                      per-layer embeddings perLayerModelProj,
//                      perLayerProjNorm, perLayerTable
// Three greedy forwards: (1) token and position as arguments; (2) the token
// the first one sampled, read on the device; (3) as (2) with the position
// read on the device, captured once as a graph and replayed. With
// cfg.fused: three steps of the fused MI355X step (encodeFusedStep twice,
// then captureFusedStep replayed once). Writes
// <dir>/out.bin: per forward hidden f32[H], logits f32[V], token u32.
// With cfg.generate = n: HipBackend.generate's pipelined greedy loop for n
// tokens at depth 2 and again at depth 1; out.bin: the u32 tokens of both.
// With cfg.prefill = [tokens]: HipBackend.prefill of those tokens from
// `position` in chunks of cfg.rows, then one fused step from its sample;
// out.bin: the sample u32, every producer layer's K then V rows of the
// prompt's positions (f16), and the step's hidden, logits and token.
const fs = require('fs');
const path = require('path');

const root = path.resolve(__dirname, '..', '..');
const hb = require(path.join(root, 'gemma4-webgpu_amd', 'node', 'hip_backend.js'));

const dir = process.argv[2];
const cfg = JSON.parse(fs.readFileSync(path.join(dir, 'config.json'), 'utf8'));
// cfg.gguf: the model (weights and configuration) from a GGUF file, caches zero
const be = cfg.gguf ? hb.HipBackend.fromGGUF(cfg.gguf, { maxSeqLen: cfg.maxSeqLen })
  : hb.HipBackend.open(hb.e2bConfig(cfg.overrides), { maxSeqLen: cfg.maxSeqLen });
const C = be.config;
console.log('[napi] device', JSON.stringify(be.g.deviceInfo(be.ctx)));

function upload(name) {
  const data = fs.readFileSync(path.join(dir, name + '.bin'));
  const p = be.alloc(data.length);
  be.g.upload(be.ctx, p, data, 0);
  return p;
}

if (!cfg.gguf) be.allocate();
for (let il = 0; il < C.num_layers && !cfg.gguf; il++) {
  const f = (cfg.formats || [])[il] || {};
  const t = {};
  for (const n of Object.keys(be.layerTensorBytes(il, f))) t[n] = upload('L' + il + '.' + n);
  be.setLayerWeights(il, t, f);
  if (hb.isKvProducer(C, il)) {
    const k = fs.readFileSync(path.join(dir, 'kv' + il + '.k.bin'));
    const v = fs.readFileSync(path.join(dir, 'kv' + il + '.v.bin'));
    be.g.upload(be.ctx, be.kvCaches[il].k, k, 0);
    be.g.upload(be.ctx, be.kvCaches[il].v, v, 0);
  }
}
if (!cfg.gguf) {
  const globals = { tokenEmbed: upload('tokenEmbed'), lmHead: upload('lmHead'), finalNorm: upload('finalNorm'),
    rope_freqs: upload('rope_freqs') };
  if (C.per_layer_input_dim > 0) {
    for (const n of ['perLayerModelProj', 'perLayerProjNorm', 'perLayerTable']) globals[n] = upload(n);
  }
  be.setGlobals(globals);
}

const H = C.hidden_size;
const V = C.vocab_size;
const outs = [];
function collect(i) {
  be.g.sync(be.ctx);
  const tok = be.readToken();
  console.log('[napi] forward ' + i + ': token ' + tok);
  outs.push(Buffer.from(be.readF32('hidden', H).buffer.slice(0)), Buffer.from(be.readF32('logits', V).buffer.slice(0)),
    Buffer.from(new Uint32Array([tok]).buffer));
}

const P = cfg.position;
if (cfg.prefill) {
  const T = cfg.prefill.length;
  const first = be.prefill(cfg.prefill, P, { rows: cfg.rows });
  console.log('[napi] prefill of ' + T + ' tokens in chunks of ' + cfg.rows + ': sample ' + first);
  const pos = be.g.download(be.ctx, be.workBuffers.position, 4).readUInt32LE(0);
  if (pos !== P + T) throw new Error('device position ' + pos + ', expected ' + (P + T));
  outs.push(Buffer.from(new Uint32Array([first]).buffer));
  for (let il = 0; il < C.num_layers; il++) {
    if (!hb.isKvProducer(C, il)) continue;
    const row = 2 * C.num_kv_heads * hb.headDim(C, il);
    for (const which of ['k', 'v']) outs.push(be.g.download(be.ctx, be.kvCaches[il][which], row * T, row * P));
  }
  be.encodeFusedStep();
  collect(1);
  fs.writeFileSync(path.join(dir, 'out.bin'), Buffer.concat(outs));
  be.close();
  console.log('[napi] done (prefill)');
  process.exit(0);
}
if (cfg.generate) {
  // greedy generation with the pipelined loop (depth 2: step N + 1 submitted
  // before step N's token is awaited), then again from the same token and
  // position with depth 1; out.bin: u32 tokens of both runs
  (async () => {
    const t2 = await be.generate(cfg.token, P, cfg.generate, { depth: 2 });
    const t1 = await be.generate(cfg.token, P, cfg.generate, { depth: 1 });
    console.log('[napi] generate depth 2: ' + t2.join(' ') + '; depth 1: ' + t1.join(' '));
    fs.writeFileSync(path.join(dir, 'out.bin'), Buffer.from(new Uint32Array(t2.concat(t1)).buffer));
    be.close();
    console.log('[napi] done (generate)');
    process.exit(0);
  })().catch((e) => {
    console.error(e);
    process.exit(1);
  });
} else if (cfg.fused) {
  // the fused MI355X step: twice eagerly (the second from the token the first
  // sampled, both at the device position the steps advance), then captured
  // once and replayed
  be.setToken(cfg.token);
  be.setPosition(P);
  be.encodeFusedStep();
  collect(1);
  be.encodeFusedStep();
  collect(2);
  const fg = be.captureFusedStep();
  be.g.graphLaunch(be.ctx, fg);
  collect(3);
  be.g.graphDestroy(fg);
  const fpos = be.g.download(be.ctx, be.workBuffers.position, 4).readUInt32LE(0);
  if (fpos !== P + 3) throw new Error('device position ' + fpos + ', expected ' + (P + 3));
  fs.writeFileSync(path.join(dir, 'out.bin'), Buffer.concat(outs));
  be.close();
  console.log('[napi] done (fused step)');
  process.exit(0);
}
if (!cfg.generate && !cfg.fused) {
be.forward(cfg.token, P);
collect(1);
be.encodeTransformerPass(null, P + 1, false);
be.sampleNextToken(true, false);
collect(2);
be.setPosition(P + 2);
be.g.graphBegin(be.ctx);
be.encodeTransformerPass(null, P + 2, true);
be.sampleNextToken(true, true);
const graph = be.g.graphEnd(be.ctx);
be.g.graphLaunch(be.ctx, graph);
collect(3);
be.g.graphDestroy(graph);
const pos = be.g.download(be.ctx, be.workBuffers.position, 4).readUInt32LE(0);
if (pos !== P + 3) throw new Error('device position ' + pos + ', expected ' + (P + 3));
fs.writeFileSync(path.join(dir, 'out.bin'), Buffer.concat(outs));
be.close();
console.log('[napi] done');
}
