'use strict';
// The GGUF keys of the N-API addon on the CPU (driven by tests/test_napi.py):
// `node gguf_read.js <file> [maxContextLength]` prints one JSON object with
// ggufInfo, the metadata (64-bit integers as strings), the tensor infos and
// configFromGGUF's result, for the Python side to compare with its reader.
const path = require('path');

const root = path.resolve(__dirname, '..', '..');
const hb = require(path.join(root, 'gemma4-webgpu_amd', 'node', 'hip_backend.js'));
const addon = hb.loadAddon();

const file = process.argv[2];
const g = addon.ggufOpen(file);
const info = addon.ggufInfo(g);
const meta = addon.ggufMetadata(g);
const tensors = addon.ggufTensors(g);
let config = null;
let configError = null;
try {
  config = hb.configFromGGUF(meta, process.argv[3] ? Number(process.argv[3]) : undefined);
} catch (e) {
  configError = e.message;
}
addon.ggufClose(g);
let openError = null;
try {
  addon.ggufOpen(file + '.absent');
} catch (e) {
  openError = e.code;
}
console.log(JSON.stringify({ info: info, meta: meta, tensors: tensors, config: config, configError: configError,
  openError: openError }, (k, v) => (typeof v === 'bigint' ? v.toString() : v)));
