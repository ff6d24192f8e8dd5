// HIP backend: the Backend / PlanRunner seam (src/backend.ts:14-46 of kleinhirn) on one MI355X
// through libkh_hip.so (include/kh_hip.h) and its Node-API binding kh_addon.node. Drop-in beside
// src/webgpu-backend.ts and src/wasm-backend.ts: the plans of src/plan/build.ts run unchanged; the
// library stores each plan's rows packed (cu_seqlens from the mask) and computes only the valid
// rows on hand-written gfx950 kernels.
//
// Node only (a native addon). Integration in the host repository:
//   * widen Backend.kind in src/backend.ts to 'webgpu' | 'wasm' | 'hip';
//   * let loadBackend (src/backend.ts:75-89) call loadHip when asked for the HIP backend.
// EncoderModel needs no change: one call in flight per model (src/encoder.ts:5-8) matches the
// library's one-stream-per-plan contract.

import { createRequire } from 'node:module';
import type { Backend, LoadedBackend, PlanRunner } from './backend.ts';
import type { RunInput } from './plan/executor.ts';
import type { Plan } from './plan/ir.ts';
import { readFileSync } from 'node:fs';
import { dirname, join } from 'node:path';
import { fetchShardBytes, loadWords, type Manifest } from './weights.ts';
import { legacyTable, wordsView, type WordsFetch, type WordTable } from './words.ts';

// The addon's surface (kleinhirn_amd/node/kh_addon.c); handles are opaque.
export type KhHandle = { readonly __kh: unique symbol };
export interface KhAddon {
  abiVersion(): number;
  ctxCreate(device: number): KhHandle;
  ctxDestroy(ctx: KhHandle): void;
  weightAdd(ctx: KhHandle, name: string, dtype: number, shape: number[], data: ArrayBufferView): void;
  weightBytes(ctx: KhHandle): number;
  wordsSet(ctx: KhHandle, dtype: number, rows: number, width: number, data: ArrayBufferView): void;
  planCheck(ctx: KhHandle | null, json: string): void;
  planCreate(ctx: KhHandle, json: string): KhHandle;
  planInitBuffer(plan: KhHandle, id: string, data: ArrayBufferView): void;
  planInfo(plan: KhHandle): { length: number; batch: number; markers: number; f16: number; bytes: number;
    outRows: number; outCols: number; launches: number; streams: number };
  planDestroy(plan: KhHandle): void;
  upload(plan: KhHandle, embeddings: ArrayBufferView, mask: Float32Array, typeIds: Uint32Array | null): void;
  uploadIds(plan: KhHandle, ids: Int32Array, mask: Float32Array, typeIds: Uint32Array | null): void;
  uploadMarkers(plan: KhHandle, packed: Uint32Array): void;
  uploadQtypes(plan: KhHandle, qtype: Uint32Array): void;
  run(plan: KhHandle, rows: number): void;
  readOutput(plan: KhHandle): Float32Array;
  readOutputAsync(plan: KhHandle): Promise<Float32Array>;
  lastRunMs(plan: KhHandle): number;
  manifestCheck(path: string, flags?: number): ManifestInfo;
  loadManifest(ctx: KhHandle, path: string, flags?: number): ManifestInfo;
  // kh_scores / kh_rank: the numeric steps after the plan (src/tasks.ts, src/encoder.ts:498-544)
  scores(logits: Float32Array, cols: number, kind: number): { scores: Float32Array; index: Int32Array };
  rank(scores: Float32Array): Int32Array;
  // kh_sched_*: packed batch scheduling over created plans (runIdsBatch, src/encoder.ts:380-436)
  schedCreate(plans: KhHandle[]): KhHandle;
  schedRun(s: KhHandle, ids: Int32Array, offsets: Float64Array, typeWords: Uint32Array | null, tokenBudget: number,
    cols: number): { out: Float32Array; stats: { chunks: number; sequences: number; tokens: number; wallMs: number;
      gpuMs: number; hostMs: number } };
  schedDestroy(s: KhHandle): void;
}

// kh_scores kinds: single-label softmax, multi-label sigmoid, regression, L2-normalised embedding
export const SCORES_SOFTMAX = 0;
export const SCORES_SIGMOID = 1;
export const SCORES_RAW = 2;
export const SCORES_L2 = 3;
// Julia's option probabilities (softmaxPrefix, src/julia.ts:57-65): pass the first
// min(markers, options) logits as one row
export const SCORES_OPTIONS = 4;

// kh_manifest_info (include/kh_hip.h)
export interface ManifestInfo {
  version: number; tensors: number; shards: number; wordsDtype: number; wordsRows: number;
  wordsWidth: number; tensorBytes: number; fileBytes: number; readMs: number; sha256Ms: number;
  rowsMs: number; uploadMs: number;
}

// kh_load_manifest flags
export const LOAD_NO_SHA256 = 1;
export const LOAD_CHECK_ROWS = 2;
export const LOAD_NO_WORDS = 4;

const KH_F32 = 0;
const KH_F16 = 1;
const ABI = 1;

export function loadAddon(path?: string): KhAddon {
  const req = createRequire(import.meta.url);
  const addon = req(path ?? process.env.KH_ADDON ?? 'kh_addon.node') as KhAddon;
  if (addon.abiVersion() !== ABI) throw new Error(`kh_addon ABI ${addon.abiVersion()}, expected ${ABI}`);
  return addon;
}

// The plan as the library reads it: the typed-array init tables travel through planInitBuffer.
export function planJson(plan: Plan): string {
  return JSON.stringify(plan, (key, value) => (key === 'init' ? undefined : value));
}

export class HipPlanRunner implements PlanRunner {
  readonly length: number;
  readonly batch: number;
  readonly markers: number;
  private h: KhHandle | undefined;

  constructor(private kh: KhAddon, ctx: KhHandle, private plan: Plan) {
    this.length = plan.length;
    this.batch = plan.batch;
    this.markers = plan.markers;
    const h = kh.planCreate(ctx, planJson(plan));
    try {
      for (const b of plan.buffers) if (b.init) kh.planInitBuffer(h, b.id, b.init);
    } catch (e) {
      kh.planDestroy(h);
      throw e;
    }
    this.h = h;
  }

  private handle(): KhHandle {
    if (!this.h) throw new Error('HIP plan runner used after destroy');
    return this.h;
  }

  // the native plan, for the addon's scheduler (schedCreate)
  get planHandle(): KhHandle {
    return this.handle();
  }

  get bytes(): number {
    return this.kh.planInfo(this.handle()).bytes;
  }

  upload(input: RunInput): void {
    // the reference's upload order and messages (src/plan/executor.ts:385-392)
    if (this.plan.inputs.markers) {
      if (!input.packedMarkers) throw new Error('plan needs packedMarkers');
      this.kh.uploadMarkers(this.handle(), input.packedMarkers);
    }
    if (this.plan.rowSelect) {
      // Julia: one type row per sequence (qtypes[b] ?? 0)
      const q = Array.isArray(input.qtype) ? input.qtype : [input.qtype ?? 0];
      this.kh.uploadQtypes(this.handle(), Uint32Array.from(q));
    }
    if (this.plan.inputs.typeIds && !input.typeIds) throw new Error('plan needs typeIds');
    this.kh.upload(this.handle(), input.embeddings, input.mask, input.typeIds ?? null);
  }

  // The same run by token ids instead of embedding rows: the rows come from the device word table
  // (HipBackend.setWords, or the words of loadManifest) on the GPU (kh_upload_ids). ids holds
  // length x batch entries laid out as the mask (entries under mask 0 are not read).
  uploadIds(ids: Int32Array, mask: Float32Array, typeIds?: Uint32Array | null,
    extra: Pick<RunInput, 'packedMarkers' | 'qtype'> = {}): void {
    if (this.plan.inputs.markers) {
      if (!extra.packedMarkers) throw new Error('plan needs packedMarkers');
      this.kh.uploadMarkers(this.handle(), extra.packedMarkers);
    }
    if (this.plan.rowSelect) {
      const q = Array.isArray(extra.qtype) ? extra.qtype : [extra.qtype ?? 0];
      this.kh.uploadQtypes(this.handle(), Uint32Array.from(q));
    }
    if (this.plan.inputs.typeIds && !typeIds) throw new Error('plan needs typeIds');
    this.kh.uploadIds(this.handle(), ids, mask, typeIds ?? null);
  }

  run(seqLen: number, capture?: boolean): void {
    if (capture) this.assertCapturable();
    this.kh.run(this.handle(), seqLen);
  }

  readOutput(): Promise<Float32Array> {
    return this.kh.readOutputAsync(this.handle());
  }

  readCapture(): Promise<Float32Array> {
    return Promise.reject(new Error('capture is the WebGPU f32 parity tool; the HIP runner has none'));
  }

  assertCapturable(): void {
    throw new Error('capture is the WebGPU f32 parity tool; the HIP runner has none');
  }

  // GPU milliseconds of the last run (hipEvents on the plan's stream)
  lastRunMs(): number {
    return this.kh.lastRunMs(this.handle());
  }

  destroy(): void {
    if (this.h) this.kh.planDestroy(this.h);
    this.h = undefined;
  }
}

export class HipBackend implements Backend {
  // Backend.kind widened to 'webgpu' | 'wasm' | 'hip' (the one-line edit of src/backend.ts:31 this
  // backend comes with); without it this line does not type-check, by design
  readonly kind = 'hip' as const;
  private ctx: KhHandle | undefined;

  constructor(private kh: KhAddon, device = 0) {
    this.ctx = kh.ctxCreate(device);
  }

  private context(): KhHandle {
    if (!this.ctx) throw new Error('HIP backend used after dispose');
    return this.ctx;
  }

  get weightBytes(): number {
    return this.kh.weightBytes(this.context());
  }

  addTensor(name: string, dtype: string, shape: number[], bytes: Uint8Array): void {
    if (dtype !== 'f16' && dtype !== 'f32') throw new Error(`tensor ${name}: dtype ${dtype}`);
    this.kh.weightAdd(this.context(), name, dtype === 'f16' ? KH_F16 : KH_F32, shape, bytes);
  }

  // Every tensor of a manifest directory on the local disk, checked and copied to device memory by
  // the library (kh_load_manifest), and its word table as the device word table.
  loadManifest(path: string, flags = 0): ManifestInfo {
    return this.kh.loadManifest(this.context(), path, flags);
  }

  // Device-resident word table: runs by token id gather rows on the GPU (kh_upload_ids).
  setWords(dtype: 'f16' | 'f32', rows: number, width: number, bytes: Uint8Array): void {
    this.kh.wordsSet(this.context(), dtype === 'f16' ? KH_F16 : KH_F32, rows, width, bytes);
  }

  check(plan: Plan): void {
    this.kh.planCheck(this.context(), planJson(plan));
  }

  runner(plan: Plan): HipPlanRunner {
    return new HipPlanRunner(this.kh, this.context(), plan);
  }

  // A packed plan holds any batch that fits HBM: the asked size is the fitting size.
  fitBatch(build: (batch: number) => Plan, batch: number): Plan | undefined {
    return batch > 1 ? build(batch) : undefined;
  }

  async prepare<S>(work: () => S): Promise<S> {
    return work();
  }

  call<S, R>(start: () => S, read: (started: S) => Promise<R>): Promise<R> {
    let started: S;
    try {
      started = start();
    } catch (e) {
      return Promise.reject(e);
    }
    return read(started);
  }

  info(): Record<string, unknown> {
    return { backend: 'hip', weightBytes: this.weightBytes, abi: this.kh.abiVersion() };
  }

  dispose(): void {
    if (this.ctx) this.kh.ctxDestroy(this.ctx);
    this.ctx = undefined;
  }
}

// Weights of a manifest into one HIP context (the loadGpu of src/webgpu-backend.ts:103 for HIP):
// every tensor except the word table, which stays on the host as in the other backends.
export async function loadHip(
  manifestUrl: string, manifest: Manifest, started?: Promise<WordsFetch>,
  options: { device?: number; addon?: KhAddon } = {},
): Promise<LoadedBackend> {
  const kh = options.addon ?? loadAddon();
  const fetched = await fetchShardBytes(manifestUrl, manifest);
  const backend = new HipBackend(kh, options.device ?? 0);
  const tUp = performance.now();
  try {
    for (const t of fetched.manifest.tensors) {
      if (t.keepOnCpu) continue;
      backend.addTensor(t.name, t.dtype, t.shape, new Uint8Array(fetched.shardBytes[t.shard], t.offset, t.byteLength));
    }
  } catch (e) {
    backend.dispose();
    throw e;
  }
  const uploadMs = performance.now() - tUp;
  const base = manifestUrl.slice(0, manifestUrl.lastIndexOf('/') + 1);
  const words = await loadWords(base, fetched.manifest, fetched.shardBytes, started);
  return {
    backend, words: words.table, downloadBytes: fetched.downloadBytes + words.bytes,
    timing: { fetchMs: fetched.fetchMs, bodyMs: fetched.bodyMs, sha256Ms: fetched.sha256Ms, uploadMs,
      ...words.timing },
  };
}

// A manifest directory on the local disk: the library maps the files, applies the checks of
// fetchShardBytes / fetchWords (src/weights.ts:150-173, src/words.ts:98-114) and copies every
// tensor and the word table to device memory with no JS-side copy. The host keeps its WordTable
// view of the same word rows for the reference's host gather (src/encoder.ts:273-282).
export function loadHipLocal(
  manifestPath: string, options: { device?: number; addon?: KhAddon; flags?: number } = {},
): LoadedBackend & { manifest: Manifest; info: ManifestInfo } {
  const kh = options.addon ?? loadAddon();
  const manifest = JSON.parse(readFileSync(manifestPath, 'utf8')) as Manifest;
  const backend = new HipBackend(kh, options.device ?? 0);
  let info: ManifestInfo;
  try {
    info = backend.loadManifest(manifestPath, options.flags ?? 0);
  } catch (e) {
    backend.dispose();
    throw e;
  }
  const base = dirname(manifestPath);
  const bytesOf = (b: Buffer): ArrayBuffer => b.buffer.slice(b.byteOffset, b.byteOffset + b.byteLength) as ArrayBuffer;
  let words: WordTable;
  if (manifest.words) {
    words = wordsView(bytesOf(readFileSync(join(base, manifest.words.file))), manifest.words);
  } else {
    // legacy: the keepOnCpu parts in row order (loadWords, src/weights.ts:67-90)
    const parts = manifest.tensors.filter((t) => t.keepOnCpu).sort((a, b) => (a.rowStart ?? 0) - (b.rowStart ?? 0));
    const joined = new Uint8Array(parts.reduce((n, t) => n + t.byteLength, 0));
    let at = 0;
    for (const t of parts) {
      const shard = readFileSync(join(base, manifest.shards[t.shard].file));
      joined.set(shard.subarray(t.offset, t.offset + t.byteLength), at);
      at += t.byteLength;
    }
    words = legacyTable(joined.buffer, parts[0].dtype === 'f16' ? 'f16' : 'f32', parts[0].shape[1]);
  }
  return {
    backend, words, manifest, info, downloadBytes: info.fileBytes,
    timing: { fetchMs: info.readMs, bodyMs: 0, sha256Ms: info.sha256Ms, uploadMs: info.uploadMs,
      embedJoinMs: 0, wordsFetchMs: 0, wordsSha256Ms: 0 },
  };
}
