/*
 * vsampler: token sampling for the vinfer engine on AMD Instinct MI355X (gfx950).
 *
 * A plain C ABI over hand-written HIP kernels. It replaces the body of the engine's per-token
 * sampler, src/vinfer/runtime/sampler.py:50-77 (`filtered_probs` + `sample`), with one batched
 * call over B rows, and adds what the engine names but does not implement: repetition,
 * presence and frequency penalties (server/protocol.py:133-135), min-p (protocol.py:142), an
 * inverse-CDF draw from caller-supplied uniforms, and the probability of a given draft id.
 *
 * Conventions (all entry points):
 *  - Every buffer is caller-allocated device memory; the library never allocates or frees.
 *    vsamp_sample's parameter columns, history (ids and offsets) and out_ids may also be pinned
 *    host memory mapped into the device's address space (hipHostMalloc): the kernels read and
 *    write them with plain loads and stores, so a one-row call needs no copy either way.
 *  - Work is enqueued asynchronously on `stream` (a hipStream_t; NULL = the null stream).
 *    Nothing synchronises the host.
 *  - Return 0 on success, a VSAMP_E_* code otherwise; vsamp_last_error() then describes the
 *    failure (thread-local, valid until the next call on the same thread).
 *  - Calls on different streams may run concurrently as long as they use different
 *    workspaces. The only global state is a per-device cache of the device check (gfx950 or
 *    not, compute units), filled on first use and never changed after, and the thread-local
 *    error message.
 */
#ifndef VSAMPLER_H
#define VSAMPLER_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define VSAMP_ABI_VERSION 11

/* Bytes of one row's sampling state (vsamp_sample_states), an opaque record. */
#define VSAMP_ROW_STATE_BYTES 40

/* vsamp_args.flags bits. */
#define VSAMP_HIST_RANGES 1u /* hist_offsets holds a [start, end) pair per row (see below) */
/* Split rows: vsamp_sample spreads each bf16 row of a batch of at most 128 rows (V >= 32768,
 * 16-byte aligned rows) over several workgroups, when the workspace holds
 * vsamp_split_workspace_bytes(); other calls run one workgroup per row. The results are
 * identical either way. On MI355X it is slower than whole rows at every batch measured (the
 * slices' merge needs device-scope fences), so it is off unless asked for. */
#define VSAMP_SPLIT_ROWS 2u
/* History append (with VSAMP_HIST_RANGES, vsamp_sample only): each row's drawn id is also
 * written to hist_ids[end] of its range (the entry right behind the ids it was penalised by),
 * so a decode loop's history grows on the device without a call of its own. hist_ids must be
 * writable and hold that entry; no row's range may contain another row's end. No reference
 * counterpart: for callers that keep per-row histories on the device (a batched decode loop).
 * Needs penalties on (a history and a penalty column). */
#define VSAMP_HIST_APPEND 4u

enum vsamp_dtype { VSAMP_BF16 = 0, VSAMP_F32 = 1 };

enum vsamp_status {
  VSAMP_OK = 0,
  VSAMP_E_ARG = 1,       /* a null pointer, a bad size or a stride that does not fit */
  VSAMP_E_DTYPE = 2,     /* logits dtype not in vsamp_dtype */
  VSAMP_E_HIP = 3,       /* a HIP runtime call failed */
  VSAMP_E_WORKSPACE = 4, /* workspace missing or smaller than vsamp_workspace_bytes() */
  VSAMP_E_DEVICE = 5     /* the current device is not a gfx950 GPU */
};

/*
 * One batch of B rows. Per-row parameter arrays have length B and live on the device; any of
 * them may be NULL, which means the engine's default for every row (SamplingParams defaults,
 * sampler.py:20-23): temperature 1, top_k 0 (off), top_p 1 (off), min_p 0 (off), repetition 1,
 * presence 0, frequency 0 (penalties off).
 */
typedef struct vsamp_args {
  /* Logits [B, V] in `dtype`; row r starts at element r * row_stride. */
  const void* logits;
  int32_t dtype; /* enum vsamp_dtype */
  int32_t batch; /* B >= 0 */
  int32_t vocab; /* V >= 1 */
  int32_t reserved0;
  int64_t row_stride; /* elements, >= V */

  /* Per-row sampling parameters (sampler.py:18-41 plus the extensions). */
  const float* temperature; /* 0 = greedy (argmax, sampler.py:70-71) */
  const int32_t* top_k;     /* 0 or >= V = off */
  const float* top_p;       /* in (0, 1]; 1 = off */
  const float* min_p;       /* in [0, 1]; 0 = off */
  const float* repetition_penalty;
  const float* presence_penalty;
  const float* frequency_penalty;

  /* Token histories in CSR form: row r's ids are hist_ids[hist_offsets[r] .. hist_offsets[r+1]).
   * Both NULL = empty histories. Ids outside [0, V) are ignored.
   * With VSAMP_HIST_RANGES in flags, hist_offsets holds 2B entries instead and row r's ids are
   * hist_ids[hist_offsets[2r] .. hist_offsets[2r+1]): per-row ranges in any order, e.g. one
   * fixed-size region per sequence slot of a decode batch. Ranges of different rows must not
   * overlap (a row's workspace entries sit under its own range). */
  const int32_t* hist_ids;
  const int32_t* hist_offsets; /* B + 1 entries, non-decreasing, hist_offsets[0] = 0 */
  int64_t hist_total;          /* hist_offsets[B] (with ranges: >= every end); sizes the workspace */

  /* The draw: one uniform u in [0, 1) per row (required). */
  const float* uniforms;
  /* Optional draft ids (one per row, in [0, V)); with out_draft_prob, reports the final
   * probability of that id after every filter. Both NULL or both set. */
  const int32_t* draft_ids;

  /* Outputs. */
  int32_t* out_ids;      /* [B] sampled token ids */
  float* out_draft_prob; /* [B] or NULL */

  /* Scratch of at least vsamp_workspace_bytes(batch, vocab, hist_total) bytes, 256-byte
   * aligned. May be NULL when that size is 0. */
  void* workspace;
  size_t workspace_bytes;

  uint32_t flags; /* VSAMP_HIST_RANGES, VSAMP_SPLIT_ROWS, VSAMP_HIST_APPEND, or 0 */
  uint32_t reserved1;
} vsamp_args;

/* The ABI version this library was built with (VSAMP_ABI_VERSION). */
int vsamp_abi_version(void);

/* 0 if `device` can run the kernels; otherwise a VSAMP_E_* code and, when why != NULL, a
 * NUL-terminated reason in why[0..n). Backs the backend's `supports(ctx)` check, which the
 * engine runs at startup (kernels/registry.py:38-43, :84-88). */
int vsamp_query(int device, char* why, size_t n);

/* Workspace bytes vsamp_sample / vsamp_probs / vsamp_penalized_logits need. */
size_t vsamp_workspace_bytes(int32_t batch, int32_t vocab, int64_t hist_total);

/* Workspace bytes of a vsamp_sample call with VSAMP_SPLIT_ROWS (the slice records and the rows'
 * arrival words after the above; equal to it when the batch does not split). The arrival words
 * need no clearing: each launch tags them. No counterpart in the engine. */
size_t vsamp_split_workspace_bytes(int32_t batch, int32_t vocab, int64_t hist_total);

/* Sample one token per row: penalties, temperature, top-k, softmax, min-p, top-p, then the
 * inverse-CDF draw with u over the kept tokens taken in descending probability (equal
 * probabilities: ascending id). Replaces `sample(logits, params, seed, position)`
 * (sampler.py:68-77) for B rows at once. */
int vsamp_sample(const vsamp_args* args, void* stream);

/* vsamp_sample without a caller workspace and without any allocation: for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc). No counterpart in the engine. The library's own workspace, a static 16 MiB
 * per GPU (held until the process ends), takes the place of `workspace`, which must be NULL with
 * workspace_bytes 0. Sizes whose vsamp_workspace_bytes() exceeds 16 MiB (histories beyond ~1.39 M
 * ids in all) fail with VSAMP_E_WORKSPACE. All calls on one GPU share that workspace: calls that
 * overlap on one GPU (different streams or threads) race. Results are identical to
 * vsamp_sample's. */
int vsamp_sample_noalloc(const vsamp_args* args, void* stream);

/* The final per-token probabilities [B, V] fp32 that vsamp_sample draws from (0 for dropped
 * tokens); row r at out + r * out_stride. Replaces `filtered_probs` (sampler.py:50-65), with the
 * extensions applied. `uniforms` and the outputs in `args` are not used. */
int vsamp_probs(const vsamp_args* args, float* out, int64_t out_stride, void* stream);

/* The penalised logits [B, V] fp32 (penalties only, no temperature); row r at
 * out + r * out_stride. Optional `counts` [B, V] int32 receives the history count of every id
 * (row r at counts + r * out_stride), or NULL. */
int vsamp_penalized_logits(const vsamp_args* args, float* out, int32_t* counts,
                           int64_t out_stride, void* stream);

/*
 * Speculative-decoding verify for B sequences with K drafted tokens each (an MTP head or a draft
 * model proposed them). Draft j of sequence b is accepted when u_accept[b, j] * q < p, p and q
 * being the target's and the draft's final probabilities of that token (every filter applied,
 * as vsamp_probs computes them); at the first rejection the emitted token is drawn with
 * u_residual[b, j] from max(0, p - q) over ascending ids (in the kernels' fixed point: token masses
 * P = rint(p~ * 2^42), kept mass S, weights (P_t * S_d >> s) - (P_d * S_t >> s)); when all
 * K are accepted the target's draw at position K (its uniform: target.uniforms of that row) is
 * the bonus token. Emitted tokens are then distributed exactly as the target's distribution.
 *
 * target: B * (K + 1) rows, row b * (K + 1) + j = the target's logits at draft position j
 * (j = K: the position after the last draft). draft: B * K rows, row b * K + j = the draft
 * distribution that proposed draft j. In both, the parameter arrays and uniforms hold ONE entry
 * per sequence (B), which applies to all of its rows; target.uniforms[b] draws the bonus token
 * (and the replacement when a residual is empty), draft.uniforms is optional and unused.
 * Both: the same vocab and dtype; no penalties (hist_ids NULL); draft_ids, out_ids and
 * out_draft_prob NULL (the call uses its workspace). Replaces nothing in the engine, which skips its checkpoint's MTP head
 * (src/vinfer/models/loader.py:27); the C5 verify workload (draft-id probability) feeds it.
 */
typedef struct vsamp_verify_args {
  vsamp_args target;
  vsamp_args draft;
  int32_t batch;     /* B */
  int32_t num_draft; /* K, 1 <= K <= 64 */
  const int32_t* draft_tokens; /* [B, K] */
  const float* u_accept;       /* [B, K] in [0, 1) */
  const float* u_residual;     /* [B, K] in [0, 1) */
  int32_t* out_tokens;         /* [B, K + 1]: the emitted tokens, then -1 */
  int32_t* out_count;          /* [B]: tokens emitted, 1 .. K + 1 (accepted drafts + 1) */
  void* workspace;             /* vsamp_verify_workspace_bytes(B, K) bytes, 256-byte aligned */
  size_t workspace_bytes;
  /* Optional: the draft rows' states [B * K] (row b * K + j), as vsamp_sample_states wrote them
   * when the drafts were drawn, with the same parameters; then the draft rows are not sampled
   * again (their logits are still read where a residual is drawn). NULL: computed here. */
  const void* draft_states;
} vsamp_verify_args;

size_t vsamp_verify_workspace_bytes(int32_t batch, int32_t num_draft);

/* vsamp_sample, and each row's sampling state (VSAMP_ROW_STATE_BYTES per row, out_states +
 * r * VSAMP_ROW_STATE_BYTES, 8-byte aligned) for a later vsamp_verify of those rows as drafts.
 * No penalties. */
int vsamp_sample_states(const vsamp_args* args, void* out_states, void* stream);

int vsamp_verify(const vsamp_verify_args* args, void* stream);

/* Log-probabilities of the raw logits (the log-softmax of the model's output, before penalties,
 * temperature and filters, as OpenAI-style `logprobs` / `top_logprobs` report them): for each
 * row, out_token_logprob[r] = logprob of tokens[r] (NaN outside [0, V)), and the row's n_top
 * largest logits (descending, ties by ascending id) as out_top_ids / out_top_logprobs
 * [B, n_top] (-1 / -inf past V). Only logits, dtype, batch, vocab and row_stride of `args` are
 * read. A row whose max logit is not finite reports NaN. n_top in [0, 32]. The engine's API
 * layer rejects these fields today (server/protocol.py:131-132). */
int vsamp_logprobs(const vsamp_args* args, const int32_t* tokens, int32_t n_top, float* out_token_logprob,
                   int32_t* out_top_ids, float* out_top_logprobs, void* stream);

/* The LM head fused with the log-softmax's statistics. */
#define VSAMP_LM_TILE 128 /* logits per statistics tile */
typedef struct vsamp_lm_head_args {
  const void* hidden; /* [batch, dim] bf16, rows 16-byte aligned */
  int64_t hidden_stride;
  const void* weight; /* [vocab, dim] bf16 (the LM head's weight), rows 16-byte aligned */
  int64_t weight_stride;
  void* logits; /* [batch, vocab] bf16, out */
  int64_t logits_stride;
  float* tile_max; /* [batch, ceil(vocab / VSAMP_LM_TILE)] each, out: per 128 logits of a row, */
  float* tile_sum; /* their max and the sum of exp(x - max) */
  int32_t batch;
  int32_t dim; /* a multiple of 64 */
  int32_t vocab;
  int32_t reserved;
} vsamp_lm_head_args;

/* logits = hidden @ weight^T with bf16 operands, fp32 accumulation and the result rounded to
 * bf16 (what `F.linear(hidden, W)` returns for bf16 tensors; replaces the engine's LM head call,
 * models/qwen/model.py:230-233), plus the per-tile statistics vsamp_logprobs_tiles takes. One
 * hand-written MFMA kernel; the logits then feed vsamp_sample as any bf16 logits do. */
int vsamp_lm_head(const vsamp_lm_head_args* args, void* stream);

/* vsamp_logprobs over bf16 logits that vsamp_lm_head wrote, with its tile statistics: the
 * normaliser comes from the statistics and the top n from the few tiles whose max can hold
 * them, instead of two passes over every row. Same outputs as vsamp_logprobs (within fp32
 * rounding of the normaliser). No counterpart in the engine (its API layer rejects logprobs,
 * server/protocol.py:131-132). */
int vsamp_logprobs_tiles(const vsamp_args* args, const float* tile_max, const float* tile_sum, const int32_t* tokens,
                         int32_t n_top, float* out_token_logprob, int32_t* out_top_ids, float* out_top_logprobs,
                         void* stream);

/* vsamp_sample over bf16 logits that vsamp_lm_head wrote, with its tile maxima (`tile_max`
 * [batch, ceil(vocab / VSAMP_LM_TILE)]: the max of every VSAMP_LM_TILE logits of a row). Same
 * outputs as vsamp_sample on the same arguments, bit for bit. Rows the maxima decide are
 * decided from a few tiles instead of a pass over the row: greedy rows (the first max lies in
 * the first tile whose max is the row max) and rows sampled with top-k <= 256 or min-p (every
 * kept token lies in a tile whose max reaches a bound taken from the maxima), without
 * penalties. Every other row (penalties, top-p alone, NaN or infinite rows, more than 64
 * candidate tiles or 256 candidate tokens) takes vsamp_sample's row passes in the same launch.
 * Replaces the sampler call after the engine's LM head (models/qwen/model.py:230-233 ->
 * runtime/sampler.py:68-77) when the LM head is vsamp_lm_head. */
int vsamp_sample_tiles(const vsamp_args* args, const float* tile_max, void* stream);

/* vsamp_sample over bf16 or fp32 logits from any source, for small batches: each row's tile maxima (the
 * max of every VSAMP_LM_TILE logits) go into `tile_max` (caller-allocated device memory,
 * [batch, ceil(vocab / VSAMP_LM_TILE)] fp32), computed by many workgroups per row, and
 * vsamp_sample_tiles runs on them. While batch * ceil(ceil(vocab / VSAMP_LM_TILE) / 64) <= 256 it
 * is one launch: a row's workgroups each write a share of its maxima and count themselves in at
 * the row's word of `arrive` (caller-allocated device memory, batch uint32 words that must be
 * zero before the first call; every call leaves them zero; calls sharing `arrive` must not run
 * at once), and the last of them finishes the row; larger batches take a launch for the maxima
 * first. Same outputs as vsamp_sample, bit for bit. One bf16 row of 151936 on one workgroup spends
 * ~10 us in its pass (an fp32 row ~20); the maxima take ~2 us over the chip, so greedy and top-k rows without penalties
 * finish sooner (the engine's per-token call, B = 1, sampler.py:68-77 via generate.py:129); other
 * rows pay the extra work. (ABI version 10: `arrive` added.) */
int vsamp_sample_tile_pass(const vsamp_args* args, float* tile_max, uint32_t* arrive, void* stream);

/* The tile statistics vsamp_lm_head writes beside its logits, for bf16 logits another GEMM wrote
 * (ABI version 11; no counterpart in the reference: it completes `F.linear(hidden, W)`,
 * models/qwen/model.py:230-233, run by the library's GEMM, which beats vsamp_lm_head's MFMA
 * tiles above 64 rows): per row of `logits` (device memory, [batch, vocab] bf16, rows
 * `row_stride` elements apart) and VSAMP_LM_TILE logits, the max (a NaN is the largest) into
 * `tile_max` and the fp32 sum of exp(x - max) over the tile (0 when the max is infinite or NaN)
 * into `tile_sum` ([batch, ceil(vocab / VSAMP_LM_TILE)] fp32 each, device memory). For
 * vsamp_logprobs_tiles and vsamp_sample_tiles. */
int vsamp_tile_stats(const void* logits, int64_t row_stride, int32_t batch, int32_t vocab, float* tile_max,
                     float* tile_sum, void* stream);

/* Host function (no device work): the draw's uniform of (seeds[i], positions[i]) into out[i],
 * i < n, all host memory. u = (splitmix64(position_seed(seed, position)) >> 40) * 2^-24, where
 * position_seed is the engine's per-token seed, sampler.py:44-47 (BLAKE2b-8 of
 * "<seed>:<position>", little-endian, top bit cleared); `uniforms` of vsamp_args takes these. */
int vsamp_uniforms(const int64_t* seeds, const int64_t* positions, int32_t n, float* out);

/* vsamp_uniforms on the device: seeds, positions and out are device memory; enqueued on `stream`
 * (ABI version 9). The same function of (seed, position), bit for bit. For decode loops whose
 * steps are replayed from a captured HIP graph: the host stages the positions, and the uniforms
 * are computed by a node of the graph instead of on the host between two replays (the engine
 * draws its per-token seeds on the host, sampler.py:44-47, one step at a time). */
int vsamp_uniforms_device(const int64_t* seeds, const int64_t* positions, int32_t n, float* out, void* stream);

/* The inputs of a speculative decode loop's next iteration, advanced on the device (ABI version 9;
 * no counterpart in the reference, whose loop runs one token at a time on the host,
 * generate.py:105-146): for loops that replay each iteration from a captured HIP graph and queue
 * the next replay before the host has read this one's tokens. `inputs` ([4 + 2 num_draft + 1, n]
 * int64, row-major, device memory): slot; last token; the token before it; that token's
 * position (position - 2, `position` being the next token's); the draft steps' positions
 * (position - 1 + j, j < num_draft); the target's positions sequence-major (entry
 * b (num_draft + 1) + c of the remaining rows: position - 1 + c). With `tokens` ([n, num_draft
 * + 1] int32) and `counts` ([n] int32: sequence b emitted its first counts[b] tokens) the inputs
 * move past that iteration (position += counts[b]); without them (both NULL) they stay. Either
 * way `uniforms` (float32, (3 num_draft + 1) n) receives the iteration's draw uniforms from the
 * sequences' `seeds` ([n] int64): the draft draws [num_draft, n] at positions -(4 (position + j)
 * + 1), acceptances and residuals [n, num_draft] at -(4 (position + j) + 2) and -(4 (position +
 * j) + 3), the bonus [n] at -(4 (position + num_draft) + 4), each as vsamp_uniforms computes it.
 * num_draft <= 21. */
int vsamp_spec_advance(int64_t* inputs, int32_t n, int32_t num_draft, const int32_t* tokens, const int32_t* counts,
                       const int64_t* seeds, float* uniforms, void* stream);

/* Description of the last failure on this thread ("" if none). */
const char* vsamp_last_error(void);

#ifdef __cplusplus
}
#endif

#endif /* VSAMPLER_H */
