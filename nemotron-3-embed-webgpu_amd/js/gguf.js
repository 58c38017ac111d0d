'use strict';
// GGUF v2/v3 reader (src/gguf/reader.ts:42-161): header, typed metadata
// (arrays nest), tensor infos, tensor data at ceil(header end / alignment),
// alignment from a number-typed general.alignment (64-bit integers read as
// BigInt do not count) or 32. Same result shape and error messages.

const GGUF_MAGIC = 0x46554747;
const GGMLType = Object.freeze({ F32: 0, F16: 1, Q4_0: 2, Q4_K: 12, Q6_K: 14 });
const ValueType = Object.freeze({ UINT8: 0, INT8: 1, UINT16: 2, INT16: 3, UINT32: 4, INT32: 5, FLOAT32: 6, BOOL: 7,
  STRING: 8, ARRAY: 9, UINT64: 10, INT64: 11, FLOAT64: 12 });

// src/gguf/reader.ts:180-210
const NEMOTRON3_METADATA_KEYS = new Set(['general.architecture', 'general.name', 'general.alignment', 'general.license',
  'general.license.name', 'general.license.link', 'mistral3.block_count', 'mistral3.context_length',
  'mistral3.embedding_length', 'mistral3.feed_forward_length', 'mistral3.attention.head_count',
  'mistral3.attention.head_count_kv', 'mistral3.attention.causal', 'mistral3.attention.key_length',
  'mistral3.attention.value_length', 'mistral3.attention.layer_norm_rms_epsilon', 'mistral3.attention.temperature_scale',
  'mistral3.rope.freq_base', 'mistral3.rope.dimension_count', 'mistral3.rope.scaling.type', 'mistral3.rope.scaling.factor',
  'mistral3.rope.scaling.original_context_length', 'mistral3.rope.scaling.yarn_beta_fast',
  'mistral3.rope.scaling.yarn_beta_slow', 'mistral3.rope.scaling.yarn_log_multiplier', 'mistral3.pooling_type',
  'tokenizer.ggml.bos_token_id', 'tokenizer.ggml.eos_token_id', 'tokenizer.ggml.padding_token_id']);

/** src/gguf/reader.ts:19-35 */
function tensorByteLength(type, elements) {
  switch (type) {
    case GGMLType.F32: return elements * 4;
    case GGMLType.F16: return elements * 2;
    case GGMLType.Q4_0:
      if (elements % 32 !== 0) throw new Error(`Q4_0 tensor has ${elements} elements, not divisible by 32`);
      return elements / 32 * 18;
    case GGMLType.Q4_K:
    case GGMLType.Q6_K: {
      const name = type === GGMLType.Q4_K ? 'Q4_K' : 'Q6_K';
      if (elements % 256 !== 0) throw new Error(`${name} tensor has ${elements} elements, not divisible by 256`);
      return elements / 256 * (type === GGMLType.Q4_K ? 144 : 210);
    }
    default:
      throw new Error(`unsupported GGML tensor type ${type}`);
  }
}

class GGUFReader {
  constructor(buffer) {
    this.buffer = buffer;
    this.view = new DataView(buffer);
    this.offset = 0;
  }

  parse(options) {
    const keys = options && options.metadataKeys;
    if (this.u32() !== GGUF_MAGIC) throw new Error('not a GGUF file');
    const version = this.u32();
    if (version < 2 || version > 3) throw new Error(`unsupported GGUF version ${version}`);
    const tensorCount = this.u64Number('tensor count');
    const metadataCount = this.u64Number('metadata count');
    const metadata = new Map();
    for (let i = 0; i < metadataCount; i += 1) {
      const key = this.string();
      const type = this.u32();
      const retain = !keys || keys.has(key);
      const value = this.value(type, retain);
      if (retain) metadata.set(key, value);
    }
    const headers = [];
    for (let i = 0; i < tensorCount; i += 1) {
      const name = this.string();
      const dimensionCount = this.u32();
      const dimensions = [];
      for (let d = 0; d < dimensionCount; d += 1) dimensions.push(this.u64Number('tensor dimension'));
      const type = this.u32();
      const offset = this.u64Number('tensor offset');
      headers.push({ name, dimensions, type, offset, elementCount: dimensions.reduce((p, v) => p * v, 1) });
    }
    const alignmentValue = metadata.get('general.alignment');
    const alignment = typeof alignmentValue === 'number' ? alignmentValue : 32;
    const dataOffset = Math.ceil(this.offset / alignment) * alignment;
    const tensors = new Map();
    for (const t of headers) {
      const byteLength = tensorByteLength(t.type, t.elementCount);
      const byteOffset = dataOffset + t.offset;
      if (byteOffset + byteLength > this.buffer.byteLength) throw new Error(`${t.name} extends past end of GGUF file`);
      tensors.set(t.name, Object.assign({}, t, { byteOffset, byteLength }));
    }
    return { version, alignment, metadata, tensors, dataOffset, buffer: this.buffer };
  }

  value(type, retain) {
    const v = this.view;
    const at = this.offset;
    const scalar = (bytes, read) => { const r = retain ? read() : undefined; this.offset += bytes; return r; };
    switch (type) {
      case ValueType.UINT8: return scalar(1, () => v.getUint8(at));
      case ValueType.INT8: return scalar(1, () => v.getInt8(at));
      case ValueType.UINT16: return scalar(2, () => v.getUint16(at, true));
      case ValueType.INT16: return scalar(2, () => v.getInt16(at, true));
      case ValueType.UINT32: return scalar(4, () => v.getUint32(at, true));
      case ValueType.INT32: return scalar(4, () => v.getInt32(at, true));
      case ValueType.FLOAT32: return scalar(4, () => v.getFloat32(at, true));
      case ValueType.BOOL: return scalar(1, () => v.getUint8(at) !== 0);
      case ValueType.STRING: { const s = this.string(); return retain ? s : undefined; }
      case ValueType.UINT64: return scalar(8, () => v.getBigUint64(at, true));
      case ValueType.INT64: return scalar(8, () => v.getBigInt64(at, true));
      case ValueType.FLOAT64: return scalar(8, () => v.getFloat64(at, true));
      case ValueType.ARRAY: {
        const elementType = this.u32();
        const length = this.u64Number('metadata array length');
        const out = retain ? new Array(length) : undefined;
        for (let i = 0; i < length; i += 1) {
          const item = this.value(elementType, retain);
          if (out) out[i] = item;
        }
        return out;
      }
      default: throw new Error(`unsupported GGUF metadata value type ${type}`);
    }
  }

  string() {
    const length = this.u64Number('string length');
    const start = this.offset;
    this.offset += length;
    return Buffer.from(this.buffer, start, length).toString('utf8');
  }

  u32() {
    const value = this.view.getUint32(this.offset, true);
    this.offset += 4;
    return value;
  }

  u64Number(label) {
    const value = this.view.getBigUint64(this.offset, true);
    this.offset += 8;
    const n = Number(value);
    if (!Number.isSafeInteger(n)) throw new Error(`${label} exceeds JavaScript's safe integer range`);
    return n;
  }
}

/** Model shape from the mistral3.* metadata and the token table (src/webgpu/model.ts:19-28 hold the same values). */
function dimsFromMetadata(model, base) {
  const md = model.metadata;
  if (md.get('general.architecture') !== 'mistral3') throw new Error('expected a mistral3 GGUF');
  const d = Object.assign({}, base);
  const num = (key, fallback) => (md.has(`mistral3.${key}`) ? Number(md.get(`mistral3.${key}`)) : fallback);
  d.hidden = num('embedding_length', d.hidden);
  d.layers = num('block_count', d.layers);
  d.qHeads = num('attention.head_count', d.qHeads);
  d.kvHeads = num('attention.head_count_kv', d.kvHeads);
  d.headDim = num('attention.key_length', d.hidden / d.qHeads);
  d.intermediate = num('feed_forward_length', d.intermediate);
  d.rmsEpsilon = num('attention.layer_norm_rms_epsilon', d.rmsEpsilon);
  d.ropeTheta = num('rope.freq_base', d.ropeTheta);
  d.mergeAfterLayer = Math.min(d.mergeAfterLayer, d.layers);
  const emb = model.tensors.get('token_embd.weight');
  if (emb) d.vocab = emb.dimensions[1];
  return d;
}

module.exports = { GGUFReader, tensorByteLength, dimsFromMetadata, NEMOTRON3_METADATA_KEYS, GGUF_VALUE_TYPE: ValueType };
