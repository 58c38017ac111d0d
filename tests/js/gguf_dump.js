'use strict';
// Prints the JS host's parse of a GGUF file as JSON (tensor table, metadata
// with BigInt as strings, dims from metadata) for the Python test to compare.
const fs = require('fs');
const path = require('path');
const host = require(path.join(__dirname, '..', '..', 'nemotron-3-embed-webgpu_amd', 'js', 'gguf'));

const file = fs.readFileSync(process.argv[2]);
const buffer = file.buffer.slice(file.byteOffset, file.byteOffset + file.byteLength);
const model = new host.GGUFReader(buffer).parse(process.argv[3] === 'filter' ? { metadataKeys: host.NEMOTRON3_METADATA_KEYS } : undefined);
const norm = (v) => (typeof v === 'bigint' ? `bigint:${v}` : Array.isArray(v) ? v.map(norm) : v);
const out = {
  version: model.version, alignment: model.alignment, dataOffset: model.dataOffset,
  metadata: Object.fromEntries(Array.from(model.metadata, ([k, v]) => [k, norm(v)])),
  tensors: Array.from(model.tensors.values()),
};
if (model.metadata.get('general.architecture') === 'mistral3') {
  out.dims = host.dimsFromMetadata(model, { hidden: 2048, qHeads: 24, kvHeads: 8, headDim: 128, intermediate: 6144,
    layers: 16, vocab: 131072, mergeAfterLayer: 4, rmsEpsilon: 1e-5, ropeTheta: 1e6, kvStrideThreshold: 2048, kvStride: 3 });
}
process.stdout.write(JSON.stringify(out));
