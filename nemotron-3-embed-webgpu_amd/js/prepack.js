'use strict';
// Offline prepack (scripts/prepack-model.ts): a Nemotron-3-Embed GGUF ->
// .wgpack with Q4_0 tile32-compact projections. Same steps and errors as the
// reference's script; requantizeMatrixToQ40 runs on the GPU through the addon
// (bit-exact with the JavaScript). The layer count comes from
// mistral3.block_count (16 in the reference's model).
//
//   node js/prepack.js [model.gguf] [model.wgpack]
const crypto = require('crypto');
const fs = require('fs');
const path = require('path');
const { native } = require('./native');
const { GGUFReader, NEMOTRON3_METADATA_KEYS } = require('./gguf');
const { buildPrepackedFile, packQ40Tile32, rawTensor } = require('./prepacked');

const QUANTIZED = [2, 12, 14];

function jsonMetadata(value) {
  const convert = (item) => {
    if (typeof item !== 'bigint') return item;
    const number = Number(item);
    if (!Number.isSafeInteger(number)) throw new Error(`metadata bigint ${item} is not safely representable`);
    return number;
  };
  return Array.isArray(value) ? value.map(convert) : convert(value);
}

/** GGUF bytes (Buffer or Uint8Array) -> .wgpack bytes. `requantize(type, bytes, k, n)` defaults to the GPU. */
function prepackGGUF(sourceFile, requantize, device) {
  const buffer = sourceFile.buffer.slice(sourceFile.byteOffset, sourceFile.byteOffset + sourceFile.byteLength);
  const gguf = new GGUFReader(buffer).parse({ metadataKeys: NEMOTRON3_METADATA_KEYS });
  if (gguf.metadata.get('general.architecture') !== 'mistral3') throw new Error('expected a mistral3 GGUF');
  let ctx = null;
  if (!requantize) {
    ctx = native().init(device === undefined ? 0 : device);
    requantize = (type, bytes, k, n) => native().requantizeQ40(ctx, type, bytes, k, n);
  }
  try {
    const sourceSha256 = crypto.createHash('sha256').update(sourceFile).digest('hex');
    const consumed = new Set();
    const part = (name) => {
      const tensor = gguf.tensors.get(name);
      if (!tensor || !QUANTIZED.includes(tensor.type) || tensor.dimensions.length !== 2) {
        throw new Error(`${name} is not a supported quantized matrix`);
      }
      consumed.add(name);
      const [k, n] = tensor.dimensions;
      const source = new Uint8Array(buffer, tensor.byteOffset, tensor.byteLength);
      return { name, k, n, bytes: requantize(tensor.type, source, k, n) };
    };
    const layers = Number(gguf.metadata.has('mistral3.block_count') ? gguf.metadata.get('mistral3.block_count') : 16);
    const packed = [];
    for (let layer = 0; layer < layers; layer += 1) {
      const p = `blk.${layer}`;
      packed.push(packQ40Tile32(`${p}.attn_qkv.weight`, [part(`${p}.attn_q.weight`), part(`${p}.attn_k.weight`), part(`${p}.attn_v.weight`)]));
      packed.push(packQ40Tile32(`${p}.attn_output.weight`, [part(`${p}.attn_output.weight`)]));
      packed.push(packQ40Tile32(`${p}.ffn_gate_up.weight`, [part(`${p}.ffn_gate.weight`), part(`${p}.ffn_up.weight`)]));
      packed.push(packQ40Tile32(`${p}.ffn_down.weight`, [part(`${p}.ffn_down.weight`)]));
    }
    const unexpected = Array.from(gguf.tensors.values()).filter((t) => t.dimensions.length === 2
      && t.name !== 'token_embd.weight' && !consumed.has(t.name));
    if (unexpected.length > 0) throw new Error(`unpacked matrices: ${unexpected.map((t) => t.name).join(', ')}`);
    const raw = Array.from(gguf.tensors.values()).filter((t) => !consumed.has(t.name))
      .map((t) => rawTensor(t.name, t.dimensions, t.type, new Uint8Array(buffer, t.byteOffset, t.byteLength)));
    const metadata = {};
    for (const [key, value] of gguf.metadata) metadata[key] = jsonMetadata(value);
    return buildPrepackedFile(sourceSha256, sourceFile.byteLength, metadata, raw.concat(packed));
  } finally {
    if (ctx) native().shutdown(ctx);
  }
}

if (require.main === module) {
  const sourcePath = process.argv[2] || 'models/nemotron-3-embed-1b-q4_k_m.gguf';
  const outputPath = process.argv[3] || 'models/nemotron-3-embed-1b-q4-webgpu.wgpack';
  const output = prepackGGUF(fs.readFileSync(sourcePath));
  fs.mkdirSync(path.dirname(path.resolve(outputPath)), { recursive: true });
  fs.writeFileSync(outputPath, output);
  console.log(JSON.stringify({ sourcePath, outputPath, bytes: output.byteLength }, null, 2));
}

module.exports = { prepackGGUF };
