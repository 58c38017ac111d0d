'use strict';
// The self-contained model pack (src/prepacked/format.ts): 8-byte magic
// WGPACK02, u32 little-endian JSON header length, the JSON header, then each
// tensor's payload at a 256-byte aligned offset from the 256-byte aligned
// data start. Tensors are 'raw' (GGUF bytes) or 'q4_0-tile32-compact'
// (20-byte records [f16 d][2 zero bytes][16 nibble bytes], ordered
// tile -> kBlock -> row32). Same checks and messages as the reference.

const MAGIC = 'WGPACK02';
const PRELUDE_BYTES = 12;
const DATA_ALIGNMENT = 256;
const PREPACKED_LAYOUT = 'q4_0-tile32-compact-v2';
const PREPACKED_TILE_ROWS = 32;
const PREPACKED_BLOCK_VALUES = 32;
const PREPACKED_BLOCK_BYTES = 20;
const PREPACKED_STORAGE_COMPACT = 'q4_0-tile32-compact';
const PREPACKED_STORAGE_RAW = 'raw';
const GGML_Q4_0 = 2;

function align(value, alignment) {
  return Math.ceil(value / alignment) * alignment;
}

/** src/prepacked/format.ts:65-99. parts: [{ name, k, n, bytes: Uint8Array }] of row-major Q4_0 blocks. */
function packQ40Tile32(name, parts) {
  if (parts.length === 0) throw new Error(`cannot pack ${name} without tensor parts`);
  const k = parts[0].k;
  if (k % PREPACKED_BLOCK_VALUES !== 0) throw new Error(`${name} K=${k} is not divisible by 32`);
  for (const part of parts) {
    if (part.k !== k) throw new Error(`${name} has mismatched K dimensions`);
    const expected = part.n * (k / 32) * 18;
    if (part.bytes.byteLength !== expected) throw new Error(`${part.name} has ${part.bytes.byteLength} bytes; expected ${expected}`);
  }
  const n = parts.reduce((sum, part) => sum + part.n, 0);
  const kBlocks = k / PREPACKED_BLOCK_VALUES;
  const tiles = Math.ceil(n / PREPACKED_TILE_ROWS);
  const out = new Uint8Array(tiles * kBlocks * PREPACKED_TILE_ROWS * PREPACKED_BLOCK_BYTES);
  // global row -> (part, row within part)
  const owner = [];
  for (const part of parts) for (let r = 0; r < part.n; r += 1) owner.push([part, r]);
  for (let row = 0; row < n; row += 1) {
    const [part, local] = owner[row];
    const tile = Math.floor(row / PREPACKED_TILE_ROWS);
    for (let kb = 0; kb < kBlocks; kb += 1) {
      const src = (local * kBlocks + kb) * 18;
      const dst = ((tile * kBlocks + kb) * PREPACKED_TILE_ROWS + (row % PREPACKED_TILE_ROWS)) * PREPACKED_BLOCK_BYTES;
      out[dst] = part.bytes[src];
      out[dst + 1] = part.bytes[src + 1];
      out.set(part.bytes.subarray(src + 2, src + 18), dst + 4);
    }
  }
  return { name, dimensions: [k, n], type: GGML_Q4_0, storage: PREPACKED_STORAGE_COMPACT, bytes: out };
}

/** src/prepacked/format.ts:101-103. */
function rawTensor(name, dimensions, type, bytes) {
  return { name, dimensions: Array.from(dimensions), type, storage: PREPACKED_STORAGE_RAW, bytes };
}

/** src/prepacked/format.ts:105-144. Returns a Uint8Array. */
function buildPrepackedFile(sourceSha256, sourceBytes, metadata, tensors) {
  let relative = 0;
  const entries = [];
  for (const tensor of tensors) {
    relative = align(relative, DATA_ALIGNMENT);
    entries.push({ name: tensor.name, dimensions: Array.from(tensor.dimensions), type: tensor.type, storage: tensor.storage,
      offset: relative, byteLength: tensor.bytes.byteLength });
    relative += tensor.bytes.byteLength;
  }
  const header = { version: 2, sourceSha256, sourceBytes, layout: PREPACKED_LAYOUT, tileRows: PREPACKED_TILE_ROWS,
    blockValues: PREPACKED_BLOCK_VALUES, blockBytes: PREPACKED_BLOCK_BYTES, metadata, tensors: entries };
  const headerBytes = Buffer.from(JSON.stringify(header), 'utf8');
  const dataOffset = align(PRELUDE_BYTES + headerBytes.byteLength, DATA_ALIGNMENT);
  const out = new Uint8Array(dataOffset + relative);
  out.set(Buffer.from(MAGIC, 'latin1'), 0);
  new DataView(out.buffer).setUint32(8, headerBytes.byteLength, true);
  out.set(headerBytes, PRELUDE_BYTES);
  tensors.forEach((tensor, i) => out.set(tensor.bytes, dataOffset + entries[i].offset));
  return out;
}

/** src/prepacked/format.ts:146-169: ArrayBuffer -> { header, tensors: Map, buffer, dataOffset }. */
function parsePrepackedModel(buffer) {
  if (buffer.byteLength < PRELUDE_BYTES) throw new Error('prepacked model is shorter than its prelude');
  const magic = Buffer.from(buffer, 0, 8).toString('latin1');
  if (magic !== MAGIC) throw new Error(`invalid prepacked model magic ${JSON.stringify(magic)}`);
  const headerLength = new DataView(buffer).getUint32(8, true);
  if (PRELUDE_BYTES + headerLength > buffer.byteLength) throw new Error('prepacked model header extends past end of file');
  const header = JSON.parse(Buffer.from(buffer, PRELUDE_BYTES, headerLength).toString('utf8'));
  if (header.version !== 2 || header.layout !== PREPACKED_LAYOUT || header.tileRows !== 32 || header.blockValues !== 32
      || header.blockBytes !== 20) {
    throw new Error(`unsupported prepacked layout ${header.layout}`);
  }
  const dataOffset = align(PRELUDE_BYTES + headerLength, DATA_ALIGNMENT);
  const tensors = new Map();
  for (const tensor of header.tensors) {
    const byteOffset = dataOffset + tensor.offset;
    if (byteOffset + tensor.byteLength > buffer.byteLength) throw new Error(`${tensor.name} extends past end of prepacked file`);
    if (tensors.has(tensor.name)) throw new Error(`duplicate prepacked tensor ${tensor.name}`);
    if (tensor.storage === PREPACKED_STORAGE_COMPACT && (tensor.type !== GGML_Q4_0 || tensor.dimensions.length !== 2)) {
      throw new Error(`${tensor.name} has invalid compact Q4_0 metadata`);
    }
    if (tensor.storage !== PREPACKED_STORAGE_COMPACT && tensor.storage !== PREPACKED_STORAGE_RAW) {
      throw new Error(`${tensor.name} has unsupported storage ${tensor.storage}`);
    }
    tensors.set(tensor.name, Object.assign({}, tensor, { byteOffset }));
  }
  return { header, tensors, buffer, dataOffset };
}

function isPrepackedModel(value) {
  return Boolean(value && value.header && value.tensors instanceof Map && value.buffer && typeof value.dataOffset === 'number');
}

module.exports = {
  MAGIC, PREPACKED_LAYOUT, PREPACKED_STORAGE_COMPACT, PREPACKED_STORAGE_RAW,
  packQ40Tile32, rawTensor, buildPrepackedFile, parsePrepackedModel, isPrepackedModel,
};
