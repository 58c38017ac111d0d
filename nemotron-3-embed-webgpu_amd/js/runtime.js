'use strict';
// The HIP runtime behind the reference's EmbeddingRuntime interface
// (src/webgpu/embedding-engine.ts:7-14): a model that createPlan()s execution
// plans whose run(ids, lengths) resolves to one L2-normalised Float32Array
// per request, computed by libnemo on an MI355X through the Node-API addon.
// Mirrors NemotronWebGPUModel / NemotronExecutionPlan (src/webgpu/model.ts).
const { native } = require('./native');
const { isPrepackedModel, PREPACKED_STORAGE_COMPACT } = require('./prepacked');

const GGMLType = Object.freeze({ F32: 0, F16: 1, Q4_0: 2, Q4_K: 12, Q6_K: 14 });
// wgpack q4_0-tile32-compact records (NEMO_TYPE_Q4_0_TILE32, include/nemo.h)
const NEMO_TYPE_Q4_0_TILE32 = 258;

/** src/webgpu/model.ts:30-32 */
function contextualMergedLength(sequence) {
  return Math.max(1, Math.ceil(sequence * 0.64));
}

/** The reference model's constants (src/webgpu/model.ts:19-28). */
function referenceDims() {
  return native().dimsReference();
}

/** The benchmark configuration's shape: 32 query heads x 64, FFN 8192. */
function configDims() {
  return Object.assign(referenceDims(), { qHeads: 32, kvHeads: 8, headDim: 64, intermediate: 8192 });
}

/** Replaces requestWebGPUDevice (src/webgpu/device.ts:6-24). */
class HipDevice {
  constructor(index) {
    this.index = index === undefined ? 0 : index;
    this.handle = native().init(this.index);
  }

  destroy() {
    if (!this.destroyed) native().shutdown(this.handle);
    this.destroyed = true;
  }
}

function requestHipDevice(index) {
  return new HipDevice(index);
}

/**
 * new NemotronHipModel(device, source, { dims, embeddingType })
 * source: a PrepackedModel (parsePrepackedModel; raw or q4_0-tile32-compact tensors), a
 * GGUF-like { tensors: Map(name -> { dimensions, type, byteOffset,
 * byteLength }), buffer }, or { synthetic: seed } for seeded synthetic weights.
 */
class NemotronHipModel {
  constructor(device, source, options) {
    const opts = options || {};
    this.device = device;
    const isGguf = source && source.metadata instanceof Map && typeof source.dataOffset === 'number' && !source.header;
    const base = isGguf && !opts.dims ? require('./gguf').dimsFromMetadata(source, referenceDims()) : referenceDims();
    this.dims = Object.assign(base, opts.dims || {});
    // No per-binding storage cap on HIP: the engine's storage split never triggers.
    this.maxStorageBufferBindingSize = undefined;
    const addon = native();
    this.handle = addon.modelCreate(device.handle, this.dims);
    try {
      if (source && source.synthetic !== undefined) {
        addon.modelSynthesize(this.handle, source.synthetic, opts.embeddingType === undefined ? GGMLType.F16 : opts.embeddingType);
      } else {
        if (!source || !(source.tensors instanceof Map)) throw new TypeError('model source must hold a tensors Map');
        for (const tensor of source.tensors.values()) {
          const compact = isPrepackedModel(source) && tensor.storage === PREPACKED_STORAGE_COMPACT;
          const bytes = new Uint8Array(source.buffer, tensor.byteOffset, tensor.byteLength);
          addon.modelSetTensor(this.handle, tensor.name, compact ? NEMO_TYPE_Q4_0_TILE32 : tensor.type, tensor.dimensions, bytes);
        }
      }
      addon.modelFinalize(this.handle);
    } catch (error) {
      addon.modelDestroy(this.handle);
      this.destroyed = true;
      throw error;
    }
  }

  createPlan(batch, sequence) {
    return new NemotronHipPlan(this, batch, sequence);
  }

  /** Fails while plans of this model are alive (destroy them first). */
  destroy() {
    if (!this.destroyed) native().modelDestroy(this.handle);
    this.destroyed = true;
  }
}

function asU32(values) {
  return values instanceof Uint32Array ? values : Uint32Array.from(values);
}

/**
 * NemotronExecutionPlan (src/webgpu/model.ts:58-234). Runs in flight are
 * counted: destroy() while some are pending closes the plan to new calls at
 * once and frees it when the last settles, so a pending run resolves
 * normally (WebGPU's destroy() is likewise safe with queued work,
 * src/webgpu/model.ts:141-144). The addon enforces the same on its handle.
 */
class NemotronHipPlan {
  constructor(model, batch, inputSequence) {
    this.model = model;
    this.batch = batch;
    this.inputSequence = inputSequence;
    this.sequence = contextualMergedLength(inputSequence);
    this.handle = native().planCreate(model.handle, batch, inputSequence);
    this.pending = 0;
    this.closed = false;
    this.destroyed = false;
  }

  /** src/webgpu/model.ts:146-176: batch fresh Float32Array(hidden), in input order. */
  run(ids, sequenceLengths) {
    if (this.closed) return Promise.reject(new Error('plan was destroyed'));
    let pending;
    try {
      pending = native().planRun(this.handle, asU32(ids), asU32(sequenceLengths));
    } catch (error) {
      return Promise.reject(error);
    }
    this.pending += 1;
    const settle = () => {
      this.pending -= 1;
      if (this.closed && this.pending === 0) this.free();
    };
    return pending.then((flat) => {
      settle();
      const hidden = flat.length / this.batch;
      const out = [];
      for (let b = 0; b < this.batch; b += 1) out.push(flat.slice(b * hidden, (b + 1) * hidden));
      return out;
    }, (error) => {
      settle();
      throw error;
    });
  }

  /** src/webgpu/model.ts:178-224: milliseconds per stage name, summed over layers. */
  profile(ids, sequenceLengths) {
    if (this.closed) return Promise.reject(new Error('plan was destroyed'));
    try {
      return Promise.resolve(native().planProfile(this.handle, asU32(ids), asU32(sequenceLengths)));
    } catch (error) {
      return Promise.reject(error);
    }
  }

  /** src/webgpu/model.ts:141-144. Later calls on the plan fail with 'plan was destroyed'. */
  destroy() {
    if (this.closed) return;
    this.closed = true;
    if (this.pending === 0) this.free();
  }

  free() {
    if (this.destroyed) return;
    this.destroyed = true;
    native().planDestroy(this.handle);
  }
}

module.exports = {
  GGMLType, contextualMergedLength, referenceDims, configDims, HipDevice, requestHipDevice, NemotronHipModel,
  NemotronHipPlan,
};
