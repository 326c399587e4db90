/**
 * TypeScript surface of the MI355X sampler: the same call surface as
 * hachiue's src/sampler.ts (SampleConfig, sampleLogits) plus batch entry
 * points.  Implemented in index.js over the Node-API addon.
 */

/** src/sampler.ts:1-7, plus optional extensions that default to off. */
export interface SampleConfig {
  temperature?: number
  topK?: number
  topP?: number
  minP?: number
  repetitionPenalty?: number
  /** extension: subtracted once from every logit whose id occurs in the history */
  presencePenalty?: number
  /** extension: subtracted n times, n = occurrences of the id in the history */
  frequencyPenalty?: number
  /** extension: value in [0, 1) used instead of Math.random() */
  uniform?: number
}

/**
 * Sample a token ID from logits with Repetition Penalty, Top-K, Top-P, Min-P
 * and Temperature (src/sampler.ts:12-17).  `logits` is updated in place with
 * the penalised values.
 */
export function sampleLogits(
  logits: Float32Array,
  vocab: number,
  history: number[] | Int32Array,
  config?: SampleConfig,
): number

export interface BatchShape {
  rows?: number
  /** floats between the starts of consecutive rows (default: vocab) */
  stride?: number
}

/** Samples every row of a [rows, stride] Float32Array in one GPU call. */
export function sampleLogitsBatch(
  logits: Float32Array,
  vocab: number,
  histories: Array<number[] | Int32Array> | null,
  configs: SampleConfig | SampleConfig[],
  uniforms?: ArrayLike<number> | null,
  shape?: BatchShape,
): Int32Array

export function sampleLogitsBatchAsync(
  logits: Float32Array,
  vocab: number,
  histories: Array<number[] | Int32Array> | null,
  configs: SampleConfig | SampleConfig[],
  uniforms?: ArrayLike<number> | null,
  shape?: BatchShape,
): Promise<Int32Array>

/** src/engine.ts:1600-1601: temperature <= 0 and no repetition penalty. */
export function isGreedyRoute(options?: SampleConfig): boolean

/**
 * The engine's GPU greedy route: the WGSL argmax of src/kernels.ts:1613-1654
 * with its tie order (equal maxima: smallest bit-reversed low byte, then the
 * smallest id; NaN and values <= -1e30 never taken).  Logits are read only.
 */
export function argmaxLogits(logits: Float32Array, vocab: number): number

export function argmaxLogitsBatch(
  logits: Float32Array,
  vocab: number,
  shape?: BatchShape,
): Int32Array

/** The engine's choice (src/engine.ts:1616-1620, :1642-1646): argmaxLogits on
 * the greedy route, sampleLogits otherwise. */
export function nextToken(
  logits: Float32Array,
  vocab: number,
  history: number[] | Int32Array,
  options?: SampleConfig,
): number

export const DEFAULTS: Readonly<Required<Pick<SampleConfig,
  'temperature' | 'topK' | 'topP' | 'minP' | 'repetitionPenalty'>>>

/** src/engine.ts:532-539 (BackendInfo): which backend a sampler runs on. */
export interface SamplerInfo {
  backend: 'hip' | 'cpu'
  label: string
  /** present when 'auto' fell back to the CPU: why the HIP backend did not start */
  fallbackReason?: string
}

export interface Sampler {
  readonly info: SamplerInfo
  sampleLogits: typeof sampleLogits
  sampleLogitsBatch: typeof sampleLogitsBatch
  sampleLogitsBatchAsync: typeof sampleLogitsBatchAsync
  isGreedyRoute: typeof isGreedyRoute
  /** on the CPU backend: the Wasm backend's greedy loop (src/wasm-backend.ts:1204-1215),
   * the first id of the largest logit above -1e30 */
  argmaxLogits: typeof argmaxLogits
  argmaxLogitsBatch: typeof argmaxLogitsBatch
  nextToken: typeof nextToken
}

/**
 * A sampler on the requested backend (src/engine.ts:521, :626-639): 'hip'
 * (default) throws when the HIP backend cannot start, 'cpu' is the
 * JavaScript sampler, 'auto' falls back to it with `info.fallbackReason`.
 */
export function createSampler(options?: { backend?: 'hip' | 'cpu' | 'auto' }): Sampler
