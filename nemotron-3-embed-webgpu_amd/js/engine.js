'use strict';
// Micro-batching of simultaneous embed() calls onto one execution plan, with
// the behaviour of NemotronEmbeddingEngine (src/webgpu/embedding-engine.ts:23-95):
// BOS prepended when missing; a flush takes up to maxBatchSize queued
// requests, fewer when the runtime's storage-binding limit or a 1500+ token
// sequence (cap 8) says so; rows are padded after each request's tokens;
// plans are cached per "batch:sequence"; a failing run rejects every request
// of its batch and the queue keeps draining.

class NemotronEmbeddingEngine {
  constructor(runtime, tokenizer, maxBatchSize, batchWindowMs, bosToken, padToken) {
    this.runtime = runtime;
    this.tokenizer = tokenizer;
    this.maxBatchSize = maxBatchSize === undefined ? 16 : maxBatchSize;
    this.batchWindowMs = batchWindowMs === undefined ? 0 : batchWindowMs;
    this.bosToken = bosToken === undefined ? 1 : bosToken;
    this.padToken = padToken === undefined ? 11 : padToken;
    if (this.maxBatchSize < 1 || this.maxBatchSize > 16) throw new Error('maxBatchSize must be between 1 and 16');
    this.pending = [];
    this.plans = new Map();
    this.scheduled = false;
    this.flushing = false;
  }

  embed(text) {
    const tokens = this.tokenizer(text).input_ids.tolist()[0].map(Number);
    if (tokens[0] !== this.bosToken) tokens.unshift(this.bosToken);
    return new Promise((resolve, reject) => {
      this.pending.push({ tokens, resolve, reject });
      this.schedule();
    });
  }

  schedule() {
    if (this.scheduled || this.flushing) return;
    this.scheduled = true;
    setTimeout(() => {
      this.scheduled = false;
      this.flush();
    }, this.batchWindowMs);
  }

  takeBatch() {
    const candidates = this.pending.slice(0, this.maxBatchSize);
    const longest = Math.max.apply(null, candidates.map((r) => r.tokens.length));
    const limit = this.runtime.maxStorageBufferBindingSize;
    const storageLimit = limit === undefined || limit === null ? Infinity : limit;
    // the largest per-request buffer of the reference's plan: gate/up, 2 x 6144 f16 per token
    const storageCap = Math.max(1, Math.floor(storageLimit / (longest * 6144 * 2 * 2)));
    const longContextCap = longest >= 1500 ? 8 : this.maxBatchSize;
    return this.pending.splice(0, Math.min(this.maxBatchSize, storageCap, longContextCap));
  }

  async flush() {
    if (this.flushing) return;
    this.flushing = true;
    try {
      while (this.pending.length > 0) {
        const requests = this.takeBatch();
        const sequence = Math.max.apply(null, requests.map((r) => r.tokens.length));
        const ids = new Uint32Array(requests.length * sequence).fill(this.padToken);
        const lengths = new Uint32Array(requests.length);
        requests.forEach((r, i) => {
          ids.set(r.tokens, i * sequence);
          lengths[i] = r.tokens.length;
        });
        const key = `${requests.length}:${sequence}`;
        let plan = this.plans.get(key);
        if (!plan) {
          plan = this.runtime.createPlan(requests.length, sequence);
          this.plans.set(key, plan);
        }
        try {
          const embeddings = await plan.run(ids, lengths);
          requests.forEach((r, i) => r.resolve(embeddings[i]));
        } catch (error) {
          requests.forEach((r) => r.reject(error));
        }
      }
    } finally {
      this.flushing = false;
      if (this.pending.length > 0) this.schedule();
    }
  }
}

module.exports = { NemotronEmbeddingEngine };
