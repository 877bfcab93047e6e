'use strict';
// Times the library's JS CPU reference of the outgoing triangle multiplication
// (triangleMultiplicationOutgoingReference, the restatement of
// webgpu/kernels/triangle/cpu-reference.js:55-99) single-threaded on the deterministic input
// of webgpu/testing/deterministic-input.js, for bench.py's CPU baseline.
//   node bench_cpu.js <length> [cHidden]   ->   {"length", "cZ", "cHidden", "seconds"}
const lf = require('./index.js');

const length = parseInt(process.argv[2] || '128', 10);
const cHidden = parseInt(process.argv[3] || '128', 10);
const input = lf.createDeterministicTriangleInput({ length: length, cZ: 128, cHidden: cHidden }, 0);
const start = process.hrtime.bigint();
const out = lf.triangleMultiplicationOutgoingReference(input);
const seconds = Number(process.hrtime.bigint() - start) / 1e9;
let finite = true;
for (let i = 0; i < out.length; i += 1) if (!Number.isFinite(out[i])) { finite = false; break; }
console.log(JSON.stringify({ length: length, cZ: 128, cHidden: cHidden, seconds: seconds, finite: finite }));
