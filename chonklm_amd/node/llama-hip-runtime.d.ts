// Type declarations of the Node host of the MI355X decode engine; the
// signatures are those of src/lib/llama-wgsl-runtime.ts (:174-324) and
// src/lib/sampling.ts (:1-7), so TypeScript callers switch by import path.

export interface ModelDef {
  id: string;
  runtime: string; // "llama-webgpu" (llama / qwen3 / gemma3 / openelm files), "gpt-webgpu" (gpt2), "lfm2-webgpu" (lfm2),
  // "granite-webgpu" (granitehybrid)
  eosIds: number[];
  vocab: number;
  layers: number;
  maxContext: number;
  base: string;
  gguf: string; // a GGUF file, or a directory holding manifest.json + NNNN.bin shards
  kvDtype?: "float16" | "float32"; // default "float16"
  defaultRepetitionPenalty?: number;
  [key: string]: unknown;
}

export interface Tokenizer {
  decode(ids: number[]): string;
}

export type ProgressCallback = (p: { loaded: number; total: number; file?: string }) => void;
export type LoadStepCallback = (s: { step: string; detail: string }) => void;

export interface RunTokenOptions {
  temperature?: number;
  topP?: number;
  topK?: number;
  repetitionPenalty?: number;
  penalizedTokenIds?: readonly number[];
  seenIds?: readonly number[];
  seed?: number; // replaces Math.random(): the draw for position p is derived from (seed, p)
}

export declare class LlamaWgslEngine {
  readonly def: ModelDef;
  runToken(tokenId: number, needLogits: boolean, opts?: RunTokenOptions): Promise<number>;
  reset(): void;
  readonly position: number;
  readLogits(): Float32Array;
  dispose(): void;
}

export interface LoadedLlamaWgslModel {
  runtime: "llama-webgpu";
  def: ModelDef;
  tokenizer: Tokenizer;
  engine: LlamaWgslEngine;
  ep: "hip";
  cachedTokenIds: number[];
  cachedNextId: number | null;
}

export interface GenerateOptions {
  maxNewTokens?: number;
  temperature?: number;
  topP?: number;
  topK?: number;
  repetitionPenalty?: number;
  seed?: number;
  onToken?: (info: { id: number; text: string; cumulative: string }) => void;
  shouldStop?: () => boolean;
}

export declare function loadLlamaWgslModel(
  model: ModelDef,
  onProgress?: ProgressCallback,
  onStep?: LoadStepCallback,
  options?: { tokenizer?: Tokenizer; device?: number },
): Promise<LoadedLlamaWgslModel>;

export declare function generateLlamaWgsl(
  loaded: LoadedLlamaWgslModel,
  promptIds: number[],
  opts?: GenerateOptions,
): Promise<{ text: string; ids: number[]; tokensPerSec: number }>;

export declare function disposeLlamaWgsl(loaded: LoadedLlamaWgslModel): void;
export declare function resetLlamaWgslConversation(loaded: LoadedLlamaWgslModel): void;

/** LoadedGptWgslModel (src/lib/gpt-wgsl-runtime.ts:120-128). */
export interface LoadedGptWgslModel extends Omit<LoadedLlamaWgslModel, "runtime"> {
  runtime: "gpt-webgpu";
}

export declare function loadGptWgslModel(
  model: ModelDef,
  onProgress?: ProgressCallback,
  onStep?: LoadStepCallback,
  options?: { tokenizer?: Tokenizer; device?: number },
): Promise<LoadedGptWgslModel>;

export declare function generateGptWgsl(
  loaded: LoadedGptWgslModel,
  promptIds: number[],
  opts?: GenerateOptions,
): Promise<{ text: string; ids: number[]; tokensPerSec: number }>;

export declare function disposeGptWgsl(loaded: LoadedGptWgslModel): void;
export declare function resetGptWgslConversation(loaded: LoadedGptWgslModel): void;

/** LoadedLfmWgslModel (src/lib/lfm-wgsl-runtime.ts:159-167). */
export interface LoadedLfmWgslModel extends Omit<LoadedLlamaWgslModel, "runtime"> {
  runtime: "lfm2-webgpu";
}

export declare function loadLfmWgslModel(
  model: ModelDef,
  onProgress?: ProgressCallback,
  onStep?: LoadStepCallback,
  options?: { tokenizer?: Tokenizer; device?: number },
): Promise<LoadedLfmWgslModel>;

export declare function generateLfmWgsl(
  loaded: LoadedLfmWgslModel,
  promptIds: number[],
  opts?: GenerateOptions,
): Promise<{ text: string; ids: number[]; tokensPerSec: number }>;

export declare function disposeLfmWgsl(loaded: LoadedLfmWgslModel): void;
export declare function resetLfmWgslConversation(loaded: LoadedLfmWgslModel): void;

/** LoadedGraniteWgslModel (src/lib/granite-wgsl-runtime.ts:158-166). */
export interface LoadedGraniteWgslModel extends Omit<LoadedLlamaWgslModel, "runtime"> {
  runtime: "granite-webgpu";
}

export declare function loadGraniteWgslModel(
  model: ModelDef,
  onProgress?: ProgressCallback,
  onStep?: LoadStepCallback,
  options?: { tokenizer?: Tokenizer; device?: number },
): Promise<LoadedGraniteWgslModel>;

export declare function generateGraniteWgsl(
  loaded: LoadedGraniteWgslModel,
  promptIds: number[],
  opts?: GenerateOptions,
): Promise<{ text: string; ids: number[]; tokensPerSec: number }>;

export declare function disposeGraniteWgsl(loaded: LoadedGraniteWgslModel): void;
export declare function resetGraniteWgslConversation(loaded: LoadedGraniteWgslModel): void;

export {
  loadLlamaWgslModel as loadPleiasWgslModel,
  generateLlamaWgsl as generatePleiasWgsl,
  disposeLlamaWgsl as disposePleiasWgsl,
  LoadedLlamaWgslModel as LoadedPleiasWgslModel,
};
