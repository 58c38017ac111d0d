'use strict';
// JavaScript host of the MI355X encoder: the reference's embedding-runtime
// API (src/webgpu/embedding-engine.ts, src/webgpu/model.ts,
// src/prepacked/format.ts) over libnemo through the Node-API addon.
const runtime = require('./runtime');
const prepacked = require('./prepacked');
const engine = require('./engine');
const gguf = require('./gguf');
const prepack = require('./prepack');
const { native, ADDON_PATH } = require('./native');

module.exports = Object.assign({ native, ADDON_PATH }, runtime, prepacked, engine, gguf, prepack);
