'use strict';
// Decode rate of HipBackend's fused step from a Node host: the E2B-shaped
// model of the decode benchmark (35 layers of hidden 1536, 8 query heads and
// 1 KV head x 256, FFN 6144, every layer owning its cache, a 512-position
// window on the local layers, Q4_K matrices with a Q6_K down projection, the
// tied Q6_K LM head over 262144 tokens; seeded synthetic weights generated on
// the device), KV caches filled to the start position, the step captured once
// and replayed. Usage: node bench_step.js [start] [steps] [warmup]; prints
// one JSON line {tok_s, us_per_token, start, steps, positions}.
const path = require('path');
const hb = require(path.join(__dirname, 'hip_backend.js'));

const start = Number(process.argv[2] || 512);
const steps = Number(process.argv[3] || 100);
const warmup = Number(process.argv[4] || 10);
const maxSeq = Math.ceil((start + warmup + steps + 64) / 256) * 256;
const C = hb.e2bConfig({ num_unshared_layers: 35, head_dim_global: 256, intermediate_unshared: 6144,
  per_layer_input_dim: 0 });
const be = hb.HipBackend.open(C, { maxSeqLen: maxSeq });
const g = be.g;
const c = be.ctx;
be.allocate();
let seed = 1000;
const H = C.hidden_size;
const q4 = (M, N) => {
  const p = be.alloc(M * N / 256 * 144);
  g.fill(c, 'q4k', p, M * N / 256, seed++);
  return p;
};
const q6 = (M, N) => {
  const p = be.alloc(M * N / 256 * 210);
  g.fill(c, 'q6k', p, M * N / 256, seed++);
  return p;
};
const f16 = (n, mean, sd) => {
  const p = be.alloc(2 * Math.max(n, 2));
  g.fill(c, 'f16', p, n, seed++, mean, sd);
  return p;
};
for (let il = 0; il < C.num_layers; il++) {
  const hd = hb.headDim(C, il);
  const Q = C.num_q_heads * hd;
  const KV = C.num_kv_heads * hd;
  const I = hb.intermediateSize(C, il);
  be.setLayerWeights(il, {
    attn_norm: f16(H, 1, 0.1), attn_q: q4(Q, H), attn_k: q4(KV, H), attn_v: q4(KV, H), attn_q_norm: f16(hd, 1, 0.1),
    attn_k_norm: f16(hd, 1, 0.1), attn_output: q4(H, Q), post_attention_norm: f16(H, 1, 0.1), ffn_norm: f16(H, 1, 0.1),
    ffn_gate: q4(I, H), ffn_up: q4(I, H), ffn_down: q6(H, I), post_ffw_norm: f16(H, 1, 0.1),
  }, {});
  const kv = be.kvCaches[il];
  g.fill(c, 'f16', kv.k, start * KV, seed++, 0, 1);
  g.fill(c, 'f16', kv.v, start * KV, seed++, 0, 1);
}
const half = C.head_dim_global / 2;
const table = new Uint16Array(half);
for (let i = 0; i < half; i++) table[i] = i < half / 4 ? 0x3c00 : 0x7c00;  // 1.0, then +Inf (no divisor past a quarter)
const rf = be.alloc(2 * half);
g.upload(c, rf, Buffer.from(table.buffer), 0);
be.setGlobals({ tokenEmbed: f16(C.vocab_size * H, 0, 0.03), lmHead: q6(C.vocab_size, H), finalNorm: f16(H, 1, 0.1),
  rope_freqs: rf, lmHeadFormat: 'q6k' });
be.setToken(1);
be.setPosition(start);
be.prepareFusedStep();
const graph = be.captureFusedStep();
for (let i = 0; i < warmup; i++) g.graphLaunch(c, graph);
g.sync(c);
const t0 = process.hrtime.bigint();
for (let i = 0; i < steps; i++) g.graphLaunch(c, graph);
g.sync(c);
const ns = Number(process.hrtime.bigint() - t0);
const end = g.download(c, be.workBuffers.position, 4).readUInt32LE(0);
g.graphDestroy(graph);
be.close();
console.log(JSON.stringify({ tok_s: Math.round(steps / (ns * 1e-9) * 10) / 10,
  us_per_token: Math.round(ns / steps / 10) / 100, start: start, steps: steps, positions: [start, end] }));
