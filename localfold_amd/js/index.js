'use strict';
// localfold-mi355x Node host: the reference's kernels-as-library classes
// (webgpu/index.js:1-8 - TriangleMultiplication{Outgoing,Incoming}Gpu, AttentionGpu,
// OuterProductMeanGpu, TransitionGpu, EvoformerBlockGpu, EvoformerStackGpu - and the AF3
// pairformer stack of webgpu/af3/trunk/pairformer-block.js:246) over the C ABI of
// include/localfold.h, reached through the N-API addon lib/localfold_napi.node.
//
// `new X(device)` takes a device from createDevice(); `run(input, options)` validates the
// input the way the reference does (RangeError with the reference's messages), copies it to
// the device, runs the HIP kernels, copies the result back and resolves to
// {output, elapsedMilliseconds, memory, kernels}.  Weights are Float32Arrays as in the
// reference, or quantised records {dtype: 'int8'|'int5'|'float16', codes, scales, zeros?,
// block} (block = flat group size, 0 = one group per output channel), decoded inside the
// kernels.  Node-12 syntax throughout (no optional chaining, no class fields).

const fs = require('fs');
const path = require('path');
const { performance } = require('perf_hooks');

let addonModule = null;
function addon() {
  if (addonModule === null) {
    // fails loudly when the addon or liblocalfold.so is missing: there is no CPU fallback
    addonModule = require(path.join(__dirname, '..', 'lib', 'localfold_napi.node'));
  }
  return addonModule;
}

const ACT = { float32: 0, float16: 1, bfloat16: 2 };
const DIRECTION = { outgoing: 0, incoming: 1 };
const BIAS = { none: 0, separate: 1, 'normalized-input': 2, logits: 3 };

// ---- device --------------------------------------------------------------------------

function createDevice(ordinal) {
  const a = addon();
  const ctx = a.contextCreate(ordinal === undefined ? 0 : ordinal);
  return {
    ctx: ctx,
    addon: a,
    resident: new WeakMap(),   // weight object -> device-resident records (uploaded once)
    profile: false,
    tail: Promise.resolve(),   // the last queued run (one run at a time per context)
    destroy: function destroy() { a.contextDestroy(ctx); },
  };
}

// ---- validation (the reference's RangeErrors) ----------------------------------------

function positiveInteger(name, value) {
  if (!Number.isSafeInteger(value) || value <= 0) {
    throw new RangeError(name + ' must be a positive safe integer; received ' + value);
  }
}

function expectLength(name, value, length) {
  const got = value === undefined || value === null ? undefined : (value.codes ? value.elements : value.length);
  if (got !== length) {
    throw new RangeError(name + ' has ' + got + ' values; expected ' + length);
  }
}

// webgpu/kernels/triangle/types.js:13-48
function validateTriangleInput(input) {
  const shape = input.shape;
  positiveInteger('length', shape.length);
  positiveInteger('cZ', shape.cZ);
  positiveInteger('cHidden', shape.cHidden);
  const pairCount = shape.length * shape.length;
  if (!Number.isSafeInteger(pairCount * Math.max(shape.cZ, shape.cHidden))) {
    throw new RangeError("tensor dimensions exceed JavaScript's safe integer range");
  }
  expectLength('z', input.z, pairCount * shape.cZ);
  expectLength('mask', input.mask, pairCount);
  const w = input.weights;
  const cZ = shape.cZ;
  const cH = shape.cHidden;
  const sizes = [
    ['layerNormInWeight', cZ], ['layerNormInBias', cZ], ['linearAPWeight', cH * cZ], ['linearAPBias', cH],
    ['linearAGWeight', cH * cZ], ['linearAGBias', cH], ['linearBPWeight', cH * cZ], ['linearBPBias', cH],
    ['linearBGWeight', cH * cZ], ['linearBGBias', cH], ['layerNormOutWeight', cH], ['layerNormOutBias', cH],
    ['linearZWeight', cZ * cH], ['linearZBias', cZ], ['linearGWeight', cZ * cZ], ['linearGBias', cZ],
  ];
  for (let i = 0; i < sizes.length; i += 1) expectLength(sizes[i][0], w[sizes[i][0]], sizes[i][1]);
  if (input.epsilon !== undefined && (!(input.epsilon > 0) || !Number.isFinite(input.epsilon))) {
    throw new RangeError('epsilon must be finite and positive; received ' + input.epsilon);
  }
}

// webgpu/kernels/attention.js:15-57
function validateAttentionInput(input) {
  const dims = [input.batch, input.queryLength, input.channels, input.heads];
  if (!dims.every(function ok(v) { return Number.isSafeInteger(v) && v > 0; })) {
    throw new RangeError('attention dimensions must be positive safe integers');
  }
  const headDim = input.headDim || input.channels / input.heads;
  if (!Number.isInteger(headDim) || headDim > 32) {
    throw new RangeError('the fused attention path requires an integral head dimension no larger than 32');
  }
  const c = input.channels;
  const projected = input.heads * headDim;
  const w = input.weights;
  const expected = [
    ['activations', input.activations, input.batch * input.queryLength * c],
    ['mask', input.mask, input.batch * input.queryLength],
    ['queryNormScale', w.queryNormScale, c], ['queryNormOffset', w.queryNormOffset, c],
    ['queryWeight', w.queryWeight, c * projected], ['keyWeight', w.keyWeight, c * projected],
    ['valueWeight', w.valueWeight, c * projected], ['gatingWeight', w.gatingWeight, c * projected],
    ['gatingBias', w.gatingBias, projected], ['outputWeight', w.outputWeight, projected * c],
    ['outputBias', w.outputBias, c],
  ];
  for (let i = 0; i < expected.length; i += 1) expectLength(expected[i][0], expected[i][1], expected[i][2]);
  const pair = input.pairBias;
  if (pair !== undefined && pair !== null && pair.source === 'separate') {
    expectLength('pair activations', pair.activations, input.queryLength * input.queryLength * pair.channels);
    expectLength('pair norm scale', pair.layerNormScale, pair.channels);
    expectLength('pair norm offset', pair.layerNormOffset, pair.channels);
    expectLength('pair projection', pair.projectionWeight, pair.channels * input.heads);
  } else if (pair !== undefined && pair !== null) {
    expectLength('normalized-input pair projection', pair.projectionWeight, c * input.heads);
  }
}

// webgpu/kernels/transition.js:445-460
function validateTransitionInput(input) {
  if (![input.rows, input.channels, input.hiddenChannels].every(function ok(v) { return Number.isSafeInteger(v) && v > 0; })) {
    throw new RangeError('transition dimensions must be positive safe integers');
  }
  const w = input.weights;
  const c = input.channels;
  const h = input.hiddenChannels;
  const lengths = [
    ['activations', input.activations, input.rows * c], ['layerNormScale', w.layerNormScale, c],
    ['layerNormOffset', w.layerNormOffset, c], ['firstWeight', w.firstWeight, c * h], ['firstBias', w.firstBias, h],
    ['secondWeight', w.secondWeight, h * c], ['secondBias', w.secondBias, c],
  ];
  for (let i = 0; i < lengths.length; i += 1) expectLength(lengths[i][0], lengths[i][1], lengths[i][2]);
}

// webgpu/kernels/outer-product-mean.js:38-70
function validateOuterProductMeanInput(input) {
  const dims = [input.sequences, input.length, input.cM, input.cOuter, input.cZ];
  if (!dims.every(function ok(v) { return Number.isSafeInteger(v) && v > 0; })) {
    throw new RangeError('outer product mean dimensions must be positive safe integers');
  }
  const w = input.weights;
  const expected = [
    ['activations', input.activations, input.sequences * input.length * input.cM],
    ['mask', input.mask, input.sequences * input.length],
    ['layerNormScale', w.layerNormScale, input.cM], ['layerNormOffset', w.layerNormOffset, input.cM],
    ['leftWeight', w.leftWeight, input.cM * input.cOuter], ['leftBias', w.leftBias, input.cOuter],
    ['rightWeight', w.rightWeight, input.cM * input.cOuter], ['rightBias', w.rightBias, input.cOuter],
    ['outputWeight', w.outputWeight, input.cOuter * input.cOuter * input.cZ], ['outputBias', w.outputBias, input.cZ],
  ];
  for (let i = 0; i < expected.length; i += 1) expectLength(expected[i][0], expected[i][1], expected[i][2]);
}

// ---- CPU reference of the outgoing update ----------------------------------------------

// webgpu/kernels/triangle/cpu-reference.js:55-99, exported as the reference exports it
// (webgpu/index.js:60) for callers that check a device result on the host.  No GPU class calls
// it.  Values are stored as float32 at the points the reference stores them (layer-norm
// outputs, each projection, the gated a/b, the contraction, the output), with double sums in
// between.  a and b are kept channel-major so that the contraction walks contiguous memory.
function triangleMultiplicationOutgoingReference(input) {
  validateTriangleInput(input);
  const n = input.shape.length;
  const cZ = input.shape.cZ;
  const cH = input.shape.cHidden;
  const eps = input.epsilon === undefined ? 1e-5 : input.epsilon;
  const w = input.weights;
  const pairs = n * n;
  const sig = function sig(x) { return 1 / (1 + Math.exp(-x)); };
  const rowNorm = function rowNorm(src, rows, c, scale, offset) {
    const dst = new Float32Array(rows * c);
    for (let r = 0; r < rows; r += 1) {
      const o = r * c;
      let sum = 0;
      for (let k = 0; k < c; k += 1) sum += src[o + k];
      const mean = sum / c;
      let sq = 0;
      for (let k = 0; k < c; k += 1) { const d = src[o + k] - mean; sq += d * d; }
      const rstd = 1 / Math.sqrt(sq / c + eps);
      for (let k = 0; k < c; k += 1) dst[o + k] = (src[o + k] - mean) * rstd * scale[k] + offset[k];
    }
    return dst;
  };
  // one (out,in) matrix row against one input row
  const dot = function dot(x, xo, m, mo, c) {
    let v = 0;
    for (let k = 0; k < c; k += 1) v += x[xo + k] * m[mo + k];
    return v;
  };
  const zn = rowNorm(input.z, pairs, cZ, w.layerNormInWeight, w.layerNormInBias);
  const a = new Float32Array(cH * pairs);
  const b = new Float32Array(cH * pairs);
  const f = Math.fround;
  for (let p = 0; p < pairs; p += 1) {
    const m = input.mask[p];
    for (let h = 0; h < cH; h += 1) {
      const ap = f(w.linearAPBias[h] + dot(zn, p * cZ, w.linearAPWeight, h * cZ, cZ));
      const ag = f(w.linearAGBias[h] + dot(zn, p * cZ, w.linearAGWeight, h * cZ, cZ));
      const bp = f(w.linearBPBias[h] + dot(zn, p * cZ, w.linearBPWeight, h * cZ, cZ));
      const bg = f(w.linearBGBias[h] + dot(zn, p * cZ, w.linearBGWeight, h * cZ, cZ));
      a[h * pairs + p] = ap * sig(ag) * m;
      b[h * pairs + p] = bp * sig(bg) * m;
    }
  }
  // x[i, j, h] = sum_k a[h, i, k] b[h, j, k]
  const x = new Float32Array(pairs * cH);
  for (let h = 0; h < cH; h += 1) {
    const base = h * pairs;
    for (let i = 0; i < n; i += 1) {
      for (let j = 0; j < n; j += 1) x[(i * n + j) * cH + h] = dot(a, base + i * n, b, base + j * n, n);
    }
  }
  const xn = rowNorm(x, pairs, cH, w.layerNormOutWeight, w.layerNormOutBias);
  const out = new Float32Array(pairs * cZ);
  for (let p = 0; p < pairs; p += 1) {
    for (let c = 0; c < cZ; c += 1) {
      const y = f(w.linearZBias[c] + dot(xn, p * cH, w.linearZWeight, c * cH, cH));
      const g = f(w.linearGBias[c] + dot(zn, p * cZ, w.linearGWeight, c * cZ, cZ));
      out[p * cZ + c] = y * sig(g);
    }
  }
  return out;
}

// webgpu/kernels/triangle/types.js:50-69, plus the relative Frobenius error
function errorMetrics(actual, expected) {
  if (actual.length !== expected.length || actual.length === 0) {
    throw new RangeError('error metrics require equally sized, non-empty arrays');
  }
  let absoluteSum = 0;
  let squareSum = 0;
  let maximum = 0;
  let expectedSquares = 0;
  for (let i = 0; i < actual.length; i += 1) {
    const delta = Math.abs(actual[i] - expected[i]);
    absoluteSum += delta;
    squareSum += delta * delta;
    expectedSquares += expected[i] * expected[i];
    maximum = Math.max(maximum, delta);
  }
  return {
    meanAbsoluteError: absoluteSum / actual.length,
    maxAbsoluteError: maximum,
    rootMeanSquareError: Math.sqrt(squareSum / actual.length),
    relativeFrobenius: Math.sqrt(squareSum) / Math.max(Math.sqrt(expectedSquares), 1e-30),
  };
}

// ---- deterministic inputs (webgpu/testing/deterministic-input.js:1-45) ----------------

function generator(seed) {
  let state = seed >>> 0;
  return function random() {
    state = (state + 0x6d2b79f5) >>> 0;
    let value = state;
    value = Math.imul(value ^ (value >>> 15), value | 1);
    value ^= value + Math.imul(value ^ (value >>> 7), value | 61);
    return ((value ^ (value >>> 14)) >>> 0) / 4294967296;
  };
}

function createDeterministicTriangleInput(shape, seed) {
  const random = generator(seed === undefined ? 7 : seed);
  const values = function values(length, scale, center) {
    const output = new Float32Array(length);
    const c = center === undefined ? 0 : center;
    for (let i = 0; i < length; i += 1) output[i] = c + (random() * 2 - 1) * scale;
    return output;
  };
  const cZ = shape.cZ;
  const cH = shape.cHidden;
  const pairs = shape.length * shape.length;
  const rz = 0.15 / Math.sqrt(cZ);
  const weights = {};
  weights.layerNormInWeight = values(cZ, 0.1, 1);
  weights.layerNormInBias = values(cZ, 0.05);
  weights.linearAPWeight = values(cH * cZ, rz);
  weights.linearAPBias = values(cH, 0.03);
  weights.linearAGWeight = values(cH * cZ, rz);
  weights.linearAGBias = values(cH, 0.03, 1);
  weights.linearBPWeight = values(cH * cZ, rz);
  weights.linearBPBias = values(cH, 0.03);
  weights.linearBGWeight = values(cH * cZ, rz);
  weights.linearBGBias = values(cH, 0.03, 1);
  weights.layerNormOutWeight = values(cH, 0.1, 1);
  weights.layerNormOutBias = values(cH, 0.05);
  weights.linearZWeight = values(cZ * cH, 0.15 / Math.sqrt(cH));
  weights.linearZBias = values(cZ, 0.03);
  weights.linearGWeight = values(cZ * cZ, rz);
  weights.linearGBias = values(cZ, 0.03, 1);
  const mask = new Float32Array(pairs);
  for (let i = 0; i < pairs; i += 1) mask[i] = random() > 0.15 ? 1 : 0;
  return { shape: shape, z: values(pairs * cZ, 1), mask: mask, weights: weights };
}

// ---- device uploads ----------------------------------------------------------------------

// One run's (or one resident weight set's) device buffers.
function Uploads(device) {
  this.device = device;
  this.buffers = [];
}
Uploads.prototype.buffer = function buffer(typed) {
  const b = this.device.addon.upload(this.device.ctx, typed);
  this.buffers.push(b);
  return b;
};
Uploads.prototype.alloc = function alloc(bytes) {
  const b = this.device.addon.alloc(this.device.ctx, bytes);
  this.buffers.push(b);
  return b;
};
Uploads.prototype.vec = function vec(values) {
  if (values === undefined || values === null) return null;
  return this.buffer(values instanceof Float32Array ? values : Float32Array.from(values));
};
// The kernels fetch int5 codes as aligned 32-bit word pairs, which reads up to 3 bytes past
// the last code byte; the reference's records carry those bytes (a slack byte, then the scale
// table), a bare code array gets 4 zero bytes appended.
function padCodes(codes) {
  const bytes = codes instanceof Uint8Array ? codes : new Uint8Array(codes.buffer, codes.byteOffset, codes.byteLength);
  const out = new Uint8Array(bytes.length + 4);
  out.set(bytes);
  return out;
}

// A weight matrix stored rows x cols in `layout` ('in_out' or 'out_in'): Float32Array values
// or a quantised record {dtype, codes, scales, zeros?, block}.
Uploads.prototype.weight = function weight(value, layout, rows, cols) {
  if (value === undefined || value === null) return null;
  if (value.codes !== undefined) {
    return {
      dtype: value.dtype, layout: layout, rows: rows, cols: cols, group: value.block || 0,
      data: this.buffer(value.dtype === 'int5' ? padCodes(value.codes) : value.codes), scales: this.buffer(value.scales),
      zeros: value.zeros ? this.buffer(value.zeros) : null,
    };
  }
  return { dtype: 'float32', layout: layout, rows: rows, cols: cols, group: 0, data: this.vec(value) };
};
Uploads.prototype.release = function release() {
  for (let i = 0; i < this.buffers.length; i += 1) this.device.addon.free(this.buffers[i]);
  this.buffers = [];
};

// Resident (cached) device weights for a host weight object: uploaded on first use.
function resident(device, key, build) {
  let entry = device.resident.get(key);
  if (entry === undefined) {
    const up = new Uploads(device);
    entry = { uploads: up, value: build(up) };
    device.resident.set(key, entry);
  }
  return entry.value;
}

function finish(device, up, outputs, start) {
  const results = outputs.map(function download(o) {
    if (o.f16) {
      const bits = new Uint16Array(o.elements);
      device.addon.download(device.ctx, o.buffer, bits);
      return float16BitsToFloat32(bits);
    }
    const host = new Float32Array(o.elements);
    device.addon.download(device.ctx, o.buffer, host);
    return host;
  });
  const elapsed = performance.now() - start;
  const kernels = device.profile ? device.addon.profileRead(device.ctx) : [];
  const memory = device.addon.memoryStats(device.ctx);
  up.release();
  return { results: results, elapsedMilliseconds: elapsed, memory: memory, kernels: kernels };
}

// ---- weight-set builders (reference names -> addon records) ------------------------------

function triangleWeights(up, w, cZ, cH) {
  return {
    lnInScale: up.vec(w.layerNormInWeight), lnInOffset: up.vec(w.layerNormInBias),
    ap: up.weight(w.linearAPWeight, 'out_in', cH, cZ), ag: up.weight(w.linearAGWeight, 'out_in', cH, cZ),
    bp: up.weight(w.linearBPWeight, 'out_in', cH, cZ), bg: up.weight(w.linearBGWeight, 'out_in', cH, cZ),
    apBias: up.vec(w.linearAPBias), agBias: up.vec(w.linearAGBias),
    bpBias: up.vec(w.linearBPBias), bgBias: up.vec(w.linearBGBias),
    lnOutScale: up.vec(w.layerNormOutWeight), lnOutOffset: up.vec(w.layerNormOutBias),
    wz: up.weight(w.linearZWeight, 'out_in', cZ, cH), wzBias: up.vec(w.linearZBias),
    wg: up.weight(w.linearGWeight, 'out_in', cZ, cZ), wgBias: up.vec(w.linearGBias),
  };
}

function attentionWeights(up, w, c, projected, pairBias, heads) {
  const out = {
    normScale: up.vec(w.queryNormScale), normOffset: up.vec(w.queryNormOffset),
    wq: up.weight(w.queryWeight, 'in_out', c, projected), wk: up.weight(w.keyWeight, 'in_out', c, projected),
    wv: up.weight(w.valueWeight, 'in_out', c, projected), wg: up.weight(w.gatingWeight, 'in_out', c, projected),
    wo: up.weight(w.outputWeight, 'in_out', projected, c),
    gBias: up.vec(w.gatingBias), oBias: up.vec(w.outputBias),
  };
  if (pairBias) {
    const pc = pairBias.source === 'separate' ? pairBias.channels : c;
    out.wb = up.weight(pairBias.projectionWeight, 'in_out', pc, heads);
    if (pairBias.source === 'separate') {
      out.pairNormScale = up.vec(pairBias.layerNormScale);
      out.pairNormOffset = up.vec(pairBias.layerNormOffset);
    }
  }
  return out;
}

function transitionWeights(up, w, c, h) {
  return {
    normScale: up.vec(w.layerNormScale), normOffset: up.vec(w.layerNormOffset),
    w1: up.weight(w.firstWeight, 'in_out', c, h), b1: up.vec(w.firstBias),
    w2: up.weight(w.secondWeight, 'in_out', h, c), b2: up.vec(w.secondBias),
  };
}

function opmWeights(up, w, cM, cOuter, cZ) {
  return {
    normScale: up.vec(w.layerNormScale), normOffset: up.vec(w.layerNormOffset),
    wl: up.weight(w.leftWeight, 'in_out', cM, cOuter), bl: up.vec(w.leftBias),
    wr: up.weight(w.rightWeight, 'in_out', cM, cOuter), br: up.vec(w.rightBias),
    wo: up.weight(w.outputWeight, 'in_out', cOuter * cOuter, cZ), bo: up.vec(w.outputBias),
  };
}

// ---- f16 storage ---------------------------------------------------------------------

// IEEE binary16 bits of each value, rounded to nearest with ties to even; overflow goes to
// infinity and NaN stays NaN (quiet).  The f32 bits are read through a Uint32Array view of
// the input's buffer (a Float32Array is always 4-byte aligned).
function float32ToFloat16Bits(values) {
  const src = values instanceof Float32Array ? values : Float32Array.from(values);
  const words = new Uint32Array(src.buffer, src.byteOffset, src.length);
  const out = new Uint16Array(src.length);
  for (let i = 0; i < words.length; i += 1) {
    const bits = words[i];
    const sign = (bits >>> 16) & 0x8000;
    const abs = bits & 0x7fffffff;
    if (abs >= 0x38800000 && abs < 0x477ff000) {
      // f16 normal range [2^-14, 65520): rebias, drop 13 bits, round up when bit 12 is set and
      // a lower bit or the kept last bit is (ties to even); a carry moves into the exponent
      out[i] = sign | (((abs - 0x38000000) >>> 13) + ((abs >>> 12) & ((abs & 0x2fff) !== 0 ? 1 : 0)));
      continue;
    }
    const exponent = (bits >>> 23) & 0xff;
    let mantissa = bits & 0x7fffff;
    const e = exponent - 112;   // the f16 exponent field (127 - 15 = 112)
    if (e > 0 && e < 0x1f) {    // [65520, 65536): rounds to infinity
      let h = (e << 10) | (mantissa >>> 13);
      const rest = mantissa & 0x1fff;
      if (rest > 0x1000 || (rest === 0x1000 && (h & 1))) h += 1;
      out[i] = sign | h;
    } else if (exponent === 0xff) {
      out[i] = sign | 0x7c00 | (mantissa ? 0x200 : 0);
    } else if (e >= 0x1f) {
      out[i] = sign | 0x7c00;
    } else if (e < -10) {
      out[i] = sign;
    } else {
      // subnormal: value = (mantissa | 2^23) * 2^(e - 14) units of 2^-24
      mantissa |= 0x800000;
      const shift = 14 - e;
      let half = mantissa >>> shift;
      const rest = mantissa & ((1 << shift) - 1), mid = 1 << (shift - 1);
      if (rest > mid || (rest === mid && (half & 1))) half += 1;
      out[i] = sign | half;
    }
  }
  return out;
}

// every binary16 value as f32, built on first use
let f16Table = null;
function float16BitsToFloat32(bits) {
  if (f16Table === null) {
    f16Table = new Float32Array(65536);
    for (let h = 0; h < 65536; h += 1) {
      const sign = (h & 0x8000) ? -1 : 1;
      const exponent = (h >>> 10) & 0x1f, mantissa = h & 0x3ff;
      if (exponent === 0) f16Table[h] = sign * mantissa * Math.pow(2, -24);
      else if (exponent === 0x1f) f16Table[h] = mantissa ? NaN : sign * Infinity;
      else f16Table[h] = sign * (1 + mantissa / 1024) * Math.pow(2, exponent - 15);
    }
  }
  const out = new Float32Array(bits.length);
  for (let i = 0; i < bits.length; i += 1) out[i] = f16Table[bits[i]];
  return out;
}

// ---- kernels-as-library classes -------------------------------------------------------

// webgpu/kernels/triangle/webgpu.js:38-169
function TriangleMultiplicationGpu(device, direction) {
  this.device = device;
  this.direction = direction;
}
// options.precision (webgpu/kernels/triangle/webgpu.js:40): 'f32' (the default) keeps z and the
// update in f32 on the device, 'f16' stores them as f16 (z rounded on upload, the update read
// back from f16); either way the kernels multiply f16 operands with f32 accumulation.
// options.variance: only the AF2 'two-pass' LayerNorm runs here (AF3's 'fast' form is the
// AF3 dialect of lf_tri_mult, which this class does not take).
TriangleMultiplicationGpu.prototype.run = function run(input, options) {
  const self = this;
  return new Promise(function execute(resolve) {
    validateTriangleInput(input);
    const precision = options && options.precision !== undefined ? options.precision : 'f32';
    if (precision !== 'f32' && precision !== 'f16') throw new RangeError('precision must be "f32" or "f16"');
    if (options && options.variance !== undefined && options.variance !== 'two-pass') {
      throw new RangeError('variance "' + options.variance + '" is not supported: this class runs the AF2 ' +
        'two-pass LayerNorm');
    }
    const dev = self.device;
    const shape = input.shape;
    const up = new Uploads(dev);
    const start = performance.now();
    if (options && options.profile) { dev.profile = true; dev.addon.profileEnable(dev.ctx, true); }
    const weights = resident(dev, input.weights, function build(wu) {
      return triangleWeights(wu, input.weights, shape.cZ, shape.cHidden);
    });
    const elements = shape.length * shape.length * shape.cZ;
    const half = precision === 'f16';
    const z = half ? up.buffer(float32ToFloat16Bits(input.z)) : up.vec(input.z);
    const out = up.alloc(elements * (half ? 2 : 4));
    dev.addon.triMult(dev.ctx, {
      direction: DIRECTION[self.direction], dialect: 0, length: shape.length, cZ: shape.cZ,
      cHidden: shape.cHidden, actDtype: half ? ACT.float16 : ACT.float32, z: z, mask: up.vec(input.mask), out: out,
      accumulate: 0, epsilon: input.epsilon === undefined ? 1e-5 : input.epsilon, weights: weights,
    });
    const r = finish(dev, up, [{ buffer: out, elements: elements, f16: half }], start);
    resolve({ output: r.results[0], elapsedMilliseconds: r.elapsedMilliseconds, memory: r.memory, kernels: r.kernels });
  });
};

function TriangleMultiplicationOutgoingGpu(device) { TriangleMultiplicationGpu.call(this, device, 'outgoing'); }
TriangleMultiplicationOutgoingGpu.prototype = Object.create(TriangleMultiplicationGpu.prototype);
function TriangleMultiplicationIncomingGpu(device) { TriangleMultiplicationGpu.call(this, device, 'incoming'); }
TriangleMultiplicationIncomingGpu.prototype = Object.create(TriangleMultiplicationGpu.prototype);

// webgpu/kernels/attention.js:2580-2739: returns the update in the activation's layout
// options (webgpu/kernels/attention.js:2586-2622: storage, flashVariant, flashPrecision,
// projectPrecision) pick among the reference's WGSL variants; there is one HIP path, so they
// are kept and have no effect
function AttentionGpu(device, options) { this.device = device; this.options = options || {}; }
AttentionGpu.prototype.run = function run(input) {
  const self = this;
  return new Promise(function execute(resolve) {
    validateAttentionInput(input);
    const dev = self.device;
    const up = new Uploads(dev);
    const start = performance.now();
    const c = input.channels;
    const headDim = input.headDim || c / input.heads;
    const pb = input.pairBias || null;
    const weights = resident(dev, input.weights, function build(wu) {
      return attentionWeights(wu, input.weights, c, input.heads * headDim, pb, input.heads);
    });
    const elements = input.batch * input.queryLength * c;
    const out = up.alloc(elements * 4);
    const args = {
      batch: input.batch, queries: input.queryLength, channels: c, heads: input.heads,
      headDim: input.headDim || 0, transpose: input.transpose ? 1 : 0, actDtype: ACT.float32,
      act: up.vec(input.activations), mask: up.vec(input.mask), out: out, accumulate: 0,
      biasMode: pb ? BIAS[pb.source] : 0, epsilon: input.epsilon === undefined ? 1e-5 : input.epsilon,
      weights: weights,
    };
    if (pb && pb.source === 'separate') {
      args.pair = up.vec(pb.activations);
      args.pairDtype = ACT.float32;
      args.pairChannels = pb.channels;
    }
    dev.addon.attention(dev.ctx, args);
    const r = finish(dev, up, [{ buffer: out, elements: elements }], start);
    resolve({ output: r.results[0], elapsedMilliseconds: r.elapsedMilliseconds, memory: r.memory, kernels: r.kernels });
  });
};

// webgpu/kernels/transition.js:1009-1105: returns the update
function TransitionGpu(device, options) { this.device = device; this.options = options || {}; }
TransitionGpu.prototype.run = function run(input) {
  const self = this;
  return new Promise(function execute(resolve) {
    validateTransitionInput(input);
    const dev = self.device;
    const up = new Uploads(dev);
    const start = performance.now();
    const weights = resident(dev, input.weights, function build(wu) {
      return transitionWeights(wu, input.weights, input.channels, input.hiddenChannels);
    });
    const elements = input.rows * input.channels;
    const out = up.alloc(elements * 4);
    dev.addon.transition(dev.ctx, {
      kind: 0, rows: input.rows, channels: input.channels, hidden: input.hiddenChannels, actDtype: ACT.float32,
      act: up.vec(input.activations), out: out, accumulate: 0,
      chunkBytes: self.options.transitionBufferLimit || 0,
      epsilon: input.epsilon === undefined ? 1e-5 : input.epsilon, weights: weights,
    });
    const r = finish(dev, up, [{ buffer: out, elements: elements }], start);
    resolve({ output: r.results[0], elapsedMilliseconds: r.elapsedMilliseconds, memory: r.memory, kernels: r.kernels });
  });
};

// webgpu/kernels/outer-product-mean.js:1748-1907: returns the pair update
function OuterProductMeanGpu(device) { this.device = device; }
OuterProductMeanGpu.prototype.run = function run(input) {
  const self = this;
  return new Promise(function execute(resolve) {
    validateOuterProductMeanInput(input);
    const dev = self.device;
    const up = new Uploads(dev);
    const start = performance.now();
    const weights = resident(dev, input.weights, function build(wu) {
      return opmWeights(wu, input.weights, input.cM, input.cOuter, input.cZ);
    });
    const elements = input.length * input.length * input.cZ;
    const out = up.alloc(elements * 4);
    dev.addon.outerProductMean(dev.ctx, {
      sequences: input.sequences, length: input.length, cM: input.cM, cOuter: input.cOuter, cZ: input.cZ,
      msaDtype: ACT.float32, msa: up.vec(input.activations), mask: up.vec(input.mask),
      pairDtype: ACT.float32, out: out, accumulate: 0,
      epsilon: input.layerNormEpsilon === undefined ? 1e-5 : input.layerNormEpsilon,
      normEpsilon: input.normalizationEpsilon === undefined ? 1e-3 : input.normalizationEpsilon,
      weights: weights,
    });
    const r = finish(dev, up, [{ buffer: out, elements: elements }], start);
    resolve({ output: r.results[0], elapsedMilliseconds: r.elapsedMilliseconds, memory: r.memory, kernels: r.kernels });
  });
};

function evoformerBlockWeights(up, w, dims) {
  const row = w.msaRowAttention;
  const col = w.msaColumnAttention;   // absent in an extra-MSA block
  const st = w.triangleAttentionStarting;
  const en = w.triangleAttentionEnding;
  // the MSA-side records are absent when only the pair halves run (ExtraMsaPairStackGpu)
  const out = {
    rowAttention: row ? attentionWeights(up, row.attention, dims.cM, dims.cM,
      { source: 'separate', channels: dims.cZ, layerNormScale: row.pairBias.layerNormScale,
        layerNormOffset: row.pairBias.layerNormOffset, projectionWeight: row.pairBias.projectionWeight }, row.heads)
      : undefined,
    rowHeads: row ? row.heads : 0,
    columnAttention: col ? attentionWeights(up, col.attention, dims.cM, dims.cM, null, col.heads) : undefined,
    columnHeads: col ? col.heads : 0,
    msaTransition: w.msaTransition ? transitionWeights(up, w.msaTransition, dims.cM, dims.msaHidden) : undefined,
    outerProductMean: opmWeights(up, w.outerProductMean, dims.cM, dims.cOuter, dims.cZ),
    triOut: triangleWeights(up, w.triangleMultiplicationOutgoing, dims.cZ, dims.triangleHidden),
    triIn: triangleWeights(up, w.triangleMultiplicationIncoming, dims.cZ, dims.triangleHidden),
    triAttStart: attentionWeights(up, st.attention, dims.cZ, dims.cZ,
      { source: 'normalized-input', projectionWeight: st.pairBias.projectionWeight }, st.heads),
    triAttStartHeads: st.heads,
    triAttEnd: attentionWeights(up, en.attention, dims.cZ, dims.cZ,
      { source: 'normalized-input', projectionWeight: en.pairBias.projectionWeight }, en.heads),
    triAttEndHeads: en.heads,
    pairTransition: transitionWeights(up, w.pairTransition, dims.cZ, dims.pairHidden),
  };
  if (!col) delete out.columnAttention;
  if (!row) delete out.rowAttention;
  if (!w.msaTransition) delete out.msaTransition;
  return out;

}

function blockDims(input, w) {
  return {
    cM: input.cM, cZ: input.cZ, cOuter: input.cOuter, triangleHidden: input.triangleHidden,
    msaHidden: input.msaHidden || (w.msaTransition ? w.msaTransition.firstBias.length : 4 * input.cM),
    pairHidden: input.pairHidden || (w.pairTransition.firstBias.length),
  };
}

// The stack runs on a libuv worker thread (the addon's call returns a promise), so the JS
// thread stays free while the GPU works; the device buffers stay referenced until it settles.
async function runEvoformer(device, input, blockWeights) {
  let up = null;
  try {
    const dims = blockDims(input, blockWeights[0]);
    up = new Uploads(device);
    const start = performance.now();
    const ws = blockWeights.map(function each(w) {
      return resident(device, w, function build(wu) { return evoformerBlockWeights(wu, w, dims); });
    });
    const msaElements = input.sequences * input.length * input.cM;
    const pairElements = input.length * input.length * input.cZ;
    expectLength('msa', input.msa, msaElements);
    expectLength('pair', input.pair, pairElements);
    const msa = up.vec(input.msa);
    const pair = up.vec(input.pair);
    await device.addon.evoformerStack(device.ctx, {
      sequences: input.sequences, length: input.length, cM: dims.cM, cZ: dims.cZ, cOuter: dims.cOuter,
      triangleHidden: dims.triangleHidden, msaHidden: dims.msaHidden, pairHidden: dims.pairHidden,
      msaDtype: ACT.float32, msa: msa, pairDtype: ACT.float32, pair: pair,
      msaMask: up.vec(input.msaMask), pairMask: up.vec(input.pairMask), epsilon: 1e-5,
    }, ws);
    const r = finish(device, up, [{ buffer: msa, elements: msaElements }, { buffer: pair, elements: pairElements }],
      start);
    return { msa: r.results[0], pair: r.results[1], elapsedMilliseconds: r.elapsedMilliseconds, memory: r.memory,
      kernels: r.kernels };
  } finally {
    if (up) up.release();
  }
}

// webgpu/af2/evoformer/block.js:1783-1824
function EvoformerBlockGpu(device) { this.device = device; }
EvoformerBlockGpu.prototype.run = function run(input) {
  return runEvoformer(this.device, input, [input.weights]);
};

// webgpu/af2/evoformer/stack.js:44-160: input.blocks is the per-block weight list
function EvoformerStackGpu(device) { this.device = device; }
EvoformerStackGpu.prototype.run = function run(input) {
  return runEvoformer(this.device, input, input.blocks);
};

// ---- AF2 extra-MSA stack ------------------------------------------------------------

// Global column attention weights (webgpu/af2/evoformer/block.js:963-980), all (in,out):
// queryWeight [cM, H*d], keyWeight / valueWeight [cM, d], gating [cM, H*d] + bias, output
// [H*d, cM] + bias, with d = gatingBias.length / heads.
function globalAttentionWeights(up, g, cM) {
  const a = g.attention;
  const hd = a.gatingBias.length;
  const d = hd / g.heads;
  return {
    normScale: up.vec(a.queryNormScale), normOffset: up.vec(a.queryNormOffset),
    wq: up.weight(a.queryWeight, 'in_out', cM, hd), wk: up.weight(a.keyWeight, 'in_out', cM, d),
    wv: up.weight(a.valueWeight, 'in_out', cM, d), wg: up.weight(a.gatingWeight, 'in_out', cM, hd),
    gBias: up.vec(a.gatingBias), wo: up.weight(a.outputWeight, 'in_out', hd, cM), oBias: up.vec(a.outputBias),
  };
}

// webgpu/af2/evoformer/stack.js:249-330: run(input) with input.blockWeights, each an
// Evoformer block's weights with msaColumnGlobalAttention in place of msaColumnAttention
// (encodeExtraMsaBlock, block.js:1715-1744); returns {msa, pair, elapsedMilliseconds, memory}.
function ExtraMsaStackGpu(device) { this.device = device; }
ExtraMsaStackGpu.prototype.run = async function run(input) {
  const device = this.device;
  let up = null;
  try {
    const blocks = input.blockWeights;
    if (!Array.isArray(blocks) || blocks.length === 0) throw new RangeError('blockWeights must be a non-empty array');
    const dims = blockDims(input, blocks[0]);
    up = new Uploads(device);
    const start = performance.now();
    const ws = blocks.map(function each(w) {
      return resident(device, w, function build(wu) {
        const e = evoformerBlockWeights(wu, w, dims);
        e.columnGlobal = globalAttentionWeights(wu, w.msaColumnGlobalAttention, dims.cM);
        e.columnGlobalHeads = w.msaColumnGlobalAttention.heads;
        return e;
      });
    });
    const msaElements = input.sequences * input.length * input.cM;
    const pairElements = input.length * input.length * input.cZ;
    expectLength('msa', input.msa, msaElements);
    expectLength('pair', input.pair, pairElements);
    const msa = up.vec(input.msa);
    const pair = up.vec(input.pair);
    await device.addon.extraMsaStack(device.ctx, {
      sequences: input.sequences, length: input.length, cM: dims.cM, cZ: dims.cZ, cOuter: dims.cOuter,
      triangleHidden: dims.triangleHidden, msaHidden: dims.msaHidden, pairHidden: dims.pairHidden,
      msaDtype: ACT.float32, msa: msa, pairDtype: ACT.float32, pair: pair,
      msaMask: up.vec(input.msaMask), pairMask: up.vec(input.pairMask), epsilon: 1e-5,
    }, ws);
    const r = finish(device, up, [{ buffer: msa, elements: msaElements }, { buffer: pair, elements: pairElements }],
      start);
    return { msa: r.results[0], pair: r.results[1], elapsedMilliseconds: r.elapsedMilliseconds, memory: r.memory,
      kernels: r.kernels };
  } finally {
    if (up) up.release();
  }
};

// ---- AF3 pairformer stack ------------------------------------------------------------

// Block weights in the CPU reference's structure (cpu/af3/trunk/pairformer.js:495-541):
// triangle projection/gate (in,out) [cZ, 2cZ] interleaved, grid attention q/k/gating (out,in)
// and v/output (in,out), SwiGLU transitions (in,out), single attention (in,out) with a q bias.
function pairformerBlockWeights(up, w, cZ, cS) {
  const tri = function tri(t) {
    return {
      lnInScale: up.vec(t.leftNormInputScale), lnInOffset: up.vec(t.leftNormInputOffset),
      ap: up.weight(t.projection, 'in_out', cZ, 2 * cZ), ag: up.weight(t.gate, 'in_out', cZ, 2 * cZ),
      lnOutScale: up.vec(t.centerNormScale), lnOutOffset: up.vec(t.centerNormOffset),
      wz: up.weight(t.outputProjection, 'in_out', cZ, cZ), wg: up.weight(t.gatingLinear, 'in_out', cZ, cZ),
    };
  };
  const grid = function grid(a) {
    const hd = a.heads * a.dimension;
    return {
      normScale: up.vec(a.actNormScale), normOffset: up.vec(a.actNormOffset),
      wq: up.weight(a.qProjection, 'out_in', hd, cZ), wk: up.weight(a.kProjection, 'out_in', hd, cZ),
      wv: up.weight(a.vProjection, 'in_out', cZ, hd), wg: up.weight(a.gatingQuery, 'out_in', hd, cZ),
      wo: up.weight(a.outputProjection, 'in_out', hd, cZ),
      gBias: up.vec(a.gatingQueryBias), oBias: up.vec(a.outputProjectionBias),
      wb: up.weight(a.pairBiasProjection, 'in_out', cZ, a.heads),
    };
  };
  const swiglu = function swiglu(t, c) {
    return {
      normScale: up.vec(t.inputLayerNormScale), normOffset: up.vec(t.inputLayerNormOffset),
      w1: up.weight(t.transition1, 'in_out', c, 8 * c), w2: up.weight(t.transition2, 'in_out', 4 * c, c),
    };
  };
  const out = {
    triOut: tri(w.triangleMultiplicationOutgoing), triIn: tri(w.triangleMultiplicationIncoming),
    attStart: grid(w.pairAttention1), attEnd: grid(w.pairAttention2), pairHeads: w.pairAttention1.heads,
    pairTransition: swiglu(w.pairTransition, cZ),
  };
  if (w.singleAttention && cS > 0) {
    const sa = w.singleAttention;
    const hd = sa.heads * sa.dimension;
    out.singleLogitsNormScale = up.vec(w.singlePairLogitsNormScale);
    out.singleLogitsNormOffset = up.vec(w.singlePairLogitsNormOffset);
    out.singleLogitsProjection = up.weight(w.singlePairLogitsProjection, 'in_out', cZ, sa.heads);
    out.singleAttention = {
      normScale: up.vec(sa.layerNormScale), normOffset: up.vec(sa.layerNormOffset),
      wq: up.weight(sa.qProjection, 'in_out', cS, hd), wk: up.weight(sa.kProjection, 'in_out', cS, hd),
      wv: up.weight(sa.vProjection, 'in_out', cS, hd), wg: up.weight(sa.gatingQuery, 'in_out', cS, hd),
      wo: up.weight(sa.outputProjection, 'in_out', hd, cS), qBias: up.vec(sa.qBias),
      wb: up.weight(w.singlePairLogitsProjection, 'in_out', cZ, sa.heads),
    };
    out.singleHeads = sa.heads;
    out.singleHeadDim = sa.dimension;
    out.singleTransition = swiglu(w.singleTransition, cS);
  }
  return out;
}

// webgpu/af2/evoformer/stack.js:163-247: run(input) with input.blockWeights, running the pair
// half of each block (encodeEvoformerPairBlock, block.js:1663-1713): the outer product mean of
// the msa, which is read and not updated, then the pair steps.  Returns {pair,
// elapsedMilliseconds, memory}.
function ExtraMsaPairStackGpu(device) { this.device = device; }
ExtraMsaPairStackGpu.prototype.run = async function run(input) {
  const device = this.device;
  let up = null;
  try {
    const blocks = input.blockWeights;
    if (!Array.isArray(blocks) || blocks.length === 0) throw new RangeError('blockWeights must be a non-empty array');
    const dims = blockDims(input, blocks[0]);
    up = new Uploads(device);
    const start = performance.now();
    const ws = blocks.map(function each(w) {
      return resident(device, w, function build(wu) { return evoformerBlockWeights(wu, w, dims); });
    });
    const msaElements = input.sequences * input.length * input.cM;
    const pairElements = input.length * input.length * input.cZ;
    expectLength('msa', input.msa, msaElements);
    expectLength('pair', input.pair, pairElements);
    const msa = up.vec(input.msa);
    const pair = up.vec(input.pair);
    await device.addon.evoformerPairStack(device.ctx, {
      sequences: input.sequences, length: input.length, cM: dims.cM, cZ: dims.cZ, cOuter: dims.cOuter,
      triangleHidden: dims.triangleHidden, msaHidden: dims.msaHidden, pairHidden: dims.pairHidden,
      msaDtype: ACT.float32, msa: msa, pairDtype: ACT.float32, pair: pair,
      msaMask: up.vec(input.msaMask), pairMask: up.vec(input.pairMask), epsilon: 1e-5,
    }, ws);
    const r = finish(device, up, [{ buffer: pair, elements: pairElements }], start);
    return { pair: r.results[0], elapsedMilliseconds: r.elapsedMilliseconds, memory: r.memory, kernels: r.kernels };
  } finally {
    if (up) up.release();
  }
};

// webgpu/af3/trunk/pairformer-block.js:246-300: run(state, blocks, dialect, options) with
// state {pair, single, pairMask, seqMask, tokens}; dialect.swapTransposedBias has no default.
function Af3PairformerStackGpu(device, options) {
  this.device = device;
  this.options = options || {};
}
Af3PairformerStackGpu.prototype.run = async function run(state, blocks, dialect, options) {
  const dev = this.device;
  const opts = options || {};
  let up = null;
  try {
    if (!dialect || typeof dialect.swapTransposedBias !== 'boolean') {
      throw new Error('dialect.swapTransposedBias has no default');
    }
    positiveInteger('tokens', state.tokens);
    const n = state.tokens;
    const cZ = state.pair.length / (n * n);
    if (!Number.isInteger(cZ) || cZ <= 0) throw new RangeError('pair has ' + state.pair.length + ' values; not tokens^2 * cZ');
    const cS = state.single ? state.single.length / n : 0;
    expectLength('pairMask', state.pairMask, n * n);
    expectLength('seqMask', state.seqMask, n);
    if (opts.variance !== undefined && opts.variance !== 'fast') {
      throw new RangeError('the pairformer runs the reference\'s fast variance; received ' + opts.variance);
    }
    up = new Uploads(dev);
    const start = performance.now();
    const pair = up.vec(state.pair);
    const single = state.single ? up.vec(state.single) : null;
    const pairMask = up.vec(state.pairMask);
    const seqMask = up.vec(state.seqMask);
    for (let b = 0; b < blocks.length; b += 1) {
      if (opts.onBlock) opts.onBlock(b);
      const w = resident(dev, blocks[b], function build(wu) { return pairformerBlockWeights(wu, blocks[b], cZ, cS); });
      await dev.addon.pairformerBlock(dev.ctx, {
        tokens: n, cZ: cZ, cS: cS, swapTransposedBias: dialect.swapTransposedBias ? 1 : 0,
        divideByLength: dialect.divideByLength ? 1 : 0, pairDtype: ACT.float32, pair: pair,
        singleDtype: ACT.float32, single: single, pairMask: pairMask, seqMask: seqMask,
        transitionChunkBytes: opts.transitionChunkBytes || 0, epsilon: opts.epsilon || 1e-5, weights: w,
      });
      if (opts.onBlockDone) opts.onBlockDone(b + 1, blocks.length);
    }
    const outs = [{ buffer: pair, elements: n * n * cZ }];
    if (single) outs.push({ buffer: single, elements: n * cS });
    const r = finish(dev, up, outs, start);
    return { pair: r.results[0], single: single ? r.results[1] : null, elapsedMilliseconds: r.elapsedMilliseconds,
      memory: r.memory, kernels: r.kernels };
  } finally {
    if (up) up.release();
  }
};

// ---- AF3 MSA module ---------------------------------------------------------------------

// cpu/af3/trunk/msa.js:233-287 block weights: outerProductMean (AF3 names), msaAttention1
// (pair-weighted averaging), msaTransition (SwiGLU) and the pairformer block's pair weights.
function msaModuleBlockWeights(up, w, cM, cZ) {
  const pf = pairformerBlockWeights(up, w, cZ, 0);
  const o = w.outerProductMean;
  const cOuter = o.outerChannels || o.leftProjection.length / cM;
  const a = w.msaAttention1;
  const hd = a.heads * a.dimension;
  return {
    opm: {
      normScale: up.vec(o.layerNormInputScale), normOffset: up.vec(o.layerNormInputOffset),
      wl: up.weight(o.leftProjection, 'in_out', cM, cOuter), wr: up.weight(o.rightProjection, 'in_out', cM, cOuter),
      wo: up.weight(o.outputW, 'in_out', cOuter * cOuter, cZ), bo: up.vec(o.outputB),
    },
    cOuter: cOuter,
    pwa: {
      actNormScale: up.vec(a.actNormScale), actNormOffset: up.vec(a.actNormOffset),
      pairNormScale: up.vec(a.pairNormScale), pairNormOffset: up.vec(a.pairNormOffset),
      pairLogits: up.weight(a.pairLogits, 'in_out', cZ, a.heads), wv: up.weight(a.vProjection, 'in_out', cM, hd),
      wg: up.weight(a.gatingQuery, 'in_out', cM, hd), wo: up.weight(a.outputProjection, 'in_out', hd, cM),
    },
    msaHeads: a.heads, msaHeadDim: a.dimension,
    msaTransition: {
      normScale: up.vec(w.msaTransition.inputLayerNormScale), normOffset: up.vec(w.msaTransition.inputLayerNormOffset),
      w1: up.weight(w.msaTransition.transition1, 'in_out', cM, 8 * cM),
      w2: up.weight(w.msaTransition.transition2, 'in_out', 4 * cM, cM),
    },
    pair: pf,
  };
}

// webgpu/af3/trunk/msa-stack.js:67-140: run(state, blocks, dialect, options) with state
// {pair, msa, pairMask, msaMask, tokens, sequences}; dialect.msaUpdateBeforeOuterProduct and
// dialect.swapTransposedBias have no default.
function Af3MsaStackGpu(device, options) {
  this.device = device;
  this.options = options || {};
}
Af3MsaStackGpu.prototype.run = async function run(state, blocks, dialect, options) {
  const dev = this.device;
  const opts = options || {};
  let up = null;
  try {
    if (!dialect || dialect.msaUpdateBeforeOuterProduct === undefined) {
      throw new Error('dialect.msaUpdateBeforeOuterProduct has no default: AF3 takes the outer product off the '
        + 'pre-update MSA and OpenDDE off the updated one');
    }
    if (dialect.swapTransposedBias === undefined) throw new Error('dialect.swapTransposedBias has no default');
    positiveInteger('tokens', state.tokens);
    positiveInteger('sequences', state.sequences);
    const n = state.tokens;
    const rows = state.sequences * n;
    const cM = blocks[0].msaChannels || opts.msaChannels || 64;
    const cZ = blocks[0].pairChannels || state.pair.length / (n * n);
    expectLength('msa', state.msa, rows * cM);
    expectLength('pair', state.pair, n * n * cZ);
    expectLength('msaMask', state.msaMask, rows);
    expectLength('pairMask', state.pairMask, n * n);
    if (opts.variance !== undefined && opts.variance !== 'fast') {
      throw new RangeError('the MSA stack runs the reference\'s fast variance; received ' + opts.variance);
    }
    up = new Uploads(dev);
    const start = performance.now();
    const msa = up.vec(state.msa);
    const pair = up.vec(state.pair);
    const msaMask = up.vec(state.msaMask);
    const pairMask = up.vec(state.pairMask);
    for (let b = 0; b < blocks.length; b += 1) {
      if (opts.onBlock) opts.onBlock(b);
      const w = resident(dev, blocks[b], function build(wu) { return msaModuleBlockWeights(wu, blocks[b], cM, cZ); });
      await dev.addon.msaModuleBlock(dev.ctx, {
        sequences: state.sequences, tokens: n, cM: cM, cZ: cZ,
        msaUpdateBeforeOuterProduct: dialect.msaUpdateBeforeOuterProduct ? 1 : 0,
        swapTransposedBias: dialect.swapTransposedBias ? 1 : 0, divideByLength: dialect.divideByLength ? 1 : 0,
        msaDtype: ACT.float32, msa: msa, pairDtype: ACT.float32, pair: pair, msaMask: msaMask, pairMask: pairMask,
        transitionChunkBytes: opts.transitionChunkBytes || 0, epsilon: opts.epsilon || 1e-5, weights: w,
      });
    }
    const r = finish(dev, up, [{ buffer: msa, elements: rows * cM }, { buffer: pair, elements: n * n * cZ }], start);
    return { msa: r.results[0], pair: r.results[1], elapsedMilliseconds: r.elapsedMilliseconds, memory: r.memory,
      kernels: r.kernels };
  } finally {
    if (up) up.release();
  }
};

// ---- AF2 input embedder ------------------------------------------------------------------

const EMBED_WEIGHT_NAMES = [
  'preprocess1dWeight', 'preprocess1dBias', 'preprocessMsaWeight', 'preprocessMsaBias', 'leftSingleWeight',
  'leftSingleBias', 'rightSingleWeight', 'rightSingleBias', 'previousPositionWeight', 'previousPositionBias',
  'previousMsaNormScale', 'previousMsaNormOffset', 'previousPairNormScale', 'previousPairNormOffset',
  'relativePositionWeight', 'relativePositionBias', 'extraMsaWeight', 'extraMsaBias',
];

// webgpu/af2/evoformer/input-embedder.js:233-356: run(input) with the reference's input
// fields; returns {msa, pairWithoutTemplates, extraMsa, elapsedMilliseconds, memory}.
function InputEmbedderGpu(device) { this.device = device; }
InputEmbedderGpu.prototype.run = function run(input) {
  const dev = this.device;
  return new Promise(function execute(resolve) {
    const L = input.length;
    positiveInteger('length', L);
    const msaElements = input.msaSequences * L * input.msaChannels;
    const pairElements = L * L * input.pairChannels;
    const extraElements = input.extraSequences * L * input.extraMsaChannels;
    expectLength('previousMsaFirstRow', input.previousMsaFirstRow, L * input.msaChannels);
    expectLength('previousPair', input.previousPair, pairElements);
    expectLength('previousPositions', input.previousPositions, L * 37 * 3);
    const weights = resident(dev, input.weights, function build(wu) {
      const o = {};
      EMBED_WEIGHT_NAMES.forEach(function each(name) { o[name] = wu.vec(input.weights[name]); });
      return o;
    });
    const up = new Uploads(dev);
    const start = performance.now();
    const msa = up.alloc(msaElements * 4);
    const pair = up.alloc(pairElements * 4);
    const extra = up.alloc(Math.max(extraElements, 1) * 4);
    dev.addon.inputEmbedder(dev.ctx, {
      length: L, msaSequences: input.msaSequences, extraSequences: input.extraSequences,
      targetChannels: input.targetChannels, msaFeatureChannels: input.msaFeatureChannels,
      msaChannels: input.msaChannels, pairChannels: input.pairChannels, extraMsaChannels: input.extraMsaChannels,
      targetFeatures: up.vec(input.targetFeatures), msaFeatures: up.vec(input.msaFeatures),
      extraMsa: up.vec(input.extraMsa), extraHasDeletion: up.vec(input.extraHasDeletion),
      extraDeletionValue: up.vec(input.extraDeletionValue), residueIndex: up.vec(input.residueIndex),
      aatype: up.vec(input.aatype), previousMsaFirstRow: up.vec(input.previousMsaFirstRow),
      previousPair: up.vec(input.previousPair), previousPositions: up.vec(input.previousPositions),
      msa: msa, pair: pair, extra: extra, weights: weights,
    });
    const outs = [{ buffer: msa, elements: msaElements }, { buffer: extra, elements: extraElements }];
    if (input.keepPair !== true) outs.push({ buffer: pair, elements: pairElements });
    const r = finish(dev, up, outs, start);
    resolve({ msa: r.results[0], extraMsa: r.results[1], pairWithoutTemplates: input.keepPair === true ? undefined : r.results[2],
      elapsedMilliseconds: r.elapsedMilliseconds, memory: r.memory, kernels: r.kernels });
  });
};

// shared/bundles/node.js:11-40: a triangle fixture directory (manifest.json + *.f32.bin)
const TRIANGLE_WEIGHT_NAMES = [
  'layerNormInWeight', 'layerNormInBias', 'linearAPWeight', 'linearAPBias', 'linearAGWeight', 'linearAGBias',
  'linearBPWeight', 'linearBPBias', 'linearBGWeight', 'linearBGBias', 'layerNormOutWeight', 'layerNormOutBias',
  'linearZWeight', 'linearZBias', 'linearGWeight', 'linearGBias',
];

function loadTriangleReferenceBundleFromFiles(manifestPath) {
  return new Promise(function load(resolve) { resolve(loadTriangleReferenceBundleFromFilesSync(manifestPath)); });
}

function loadTriangleReferenceBundleFromFilesSync(manifestPath) {
  {
    const manifest = JSON.parse(fs.readFileSync(manifestPath, 'utf8'));
    if (manifest.formatVersion !== 1 || manifest.operator !== 'TriangleMultiplicationOutgoing') {
      throw new Error('unsupported triangle reference manifest');
    }
    const directory = path.dirname(manifestPath);
    const tensor = function tensor(name) {
      const record = manifest.tensors[name];
      if (record === undefined || record.dtype !== 'float32') throw new Error('missing float32 tensor ' + name);
      const bytes = fs.readFileSync(path.resolve(directory, record.file));
      const count = record.shape.reduce(function mul(a, b) { return a * b; }, 1);
      if (bytes.byteLength !== count * 4) throw new Error('invalid byte length for tensor ' + name);
      return new Float32Array(bytes.buffer.slice(bytes.byteOffset, bytes.byteOffset + bytes.byteLength));
    };
    const weights = {};
    TRIANGLE_WEIGHT_NAMES.forEach(function each(name) { weights[name] = tensor(name); });
    return {
      source: manifest.source,
      input: { shape: manifest.shape, epsilon: manifest.epsilon, z: tensor('z'), mask: tensor('mask'), weights: weights },
      expected: tensor('expected'),
    };
  }
}

// ---- one run at a time per device -------------------------------------------------------

// A device's context serves one run at a time: the stacks run on a libuv worker thread, and a
// second run on the same context (Promise.all over two runs, say) must not upload, allocate
// or launch while the first is pending.  Every run() therefore waits for the device's
// previous run to settle (the addon also locks the context, so an unqueued call blocks
// rather than races).
function serialiseRuns(Cls) {
  const inner = Cls.prototype.run;
  Cls.prototype.run = function run() {
    const self = this;
    const args = arguments;
    const dev = this.device;
    const go = function go() { return inner.apply(self, args); };
    const p = (dev.tail || Promise.resolve()).then(go);
    dev.tail = p.then(function settled() {}, function settled() {});
    return p;
  };
}
[TriangleMultiplicationGpu, AttentionGpu, TransitionGpu, OuterProductMeanGpu, EvoformerBlockGpu, EvoformerStackGpu,
  ExtraMsaStackGpu, ExtraMsaPairStackGpu, Af3PairformerStackGpu, Af3MsaStackGpu, InputEmbedderGpu].forEach(serialiseRuns);

module.exports = {
  loadTriangleReferenceBundleFromFiles: loadTriangleReferenceBundleFromFiles,
  loadTriangleReferenceBundleFromFilesSync: loadTriangleReferenceBundleFromFilesSync,
  createDevice: createDevice,
  TriangleMultiplicationOutgoingGpu: TriangleMultiplicationOutgoingGpu,
  TriangleMultiplicationIncomingGpu: TriangleMultiplicationIncomingGpu,
  AttentionGpu: AttentionGpu,
  TransitionGpu: TransitionGpu,
  OuterProductMeanGpu: OuterProductMeanGpu,
  EvoformerBlockGpu: EvoformerBlockGpu,
  EvoformerStackGpu: EvoformerStackGpu,
  ExtraMsaStackGpu: ExtraMsaStackGpu,
  ExtraMsaPairStackGpu: ExtraMsaPairStackGpu,
  Af3PairformerStackGpu: Af3PairformerStackGpu,
  Af3MsaStackGpu: Af3MsaStackGpu,
  InputEmbedderGpu: InputEmbedderGpu,
  validateTriangleInput: validateTriangleInput,
  validateAttentionInput: validateAttentionInput,
  validateTransitionInput: validateTransitionInput,
  validateOuterProductMeanInput: validateOuterProductMeanInput,
  errorMetrics: errorMetrics,
  triangleMultiplicationOutgoingReference: triangleMultiplicationOutgoingReference,
  generator: generator,
  createDeterministicTriangleInput: createDeterministicTriangleInput,
  float32ToFloat16Bits: float32ToFloat16Bits,
  float16BitsToFloat32: float16BitsToFloat32,
  addon: addon,
};
