/* serve.c -- generation and the serve loop over a decoder's captured step.
 *
 * Reference counterpart: the serve mode of bench/dsv2_decode_bench.c
 * (:2749-2897): weights and the captured step stay resident, a prompt is
 * consumed one position at a time by replaying the step with the prompt
 * token written into the device token buffer (:2769-2779), then the step
 * replays with the device-resident token, and generation stops at the eos
 * id (not emitted) or the per-request cap.  The line protocol is the
 * reference's: "ready" once, then per request line "id,id,...[|max_new]"
 * one response line "ids: id,id,...", timing on stderr, EOF ends.
 *
 * MI355X specifics: the token and position never leave the device during
 * generation; the host reads the generated ids back in bursts of up to 8
 * replays (one synchronisation per burst, not per token) from the history
 * buffer the argmax / sampling kernel fills. */
#define _GNU_SOURCE
#include "internal.h"

#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>
#include <unistd.h>

static double now_ms(void) {
  struct timespec ts;
  clock_gettime(CLOCK_MONOTONIC, &ts);
  return (double)ts.tv_sec * 1e3 + (double)ts.tv_nsec / 1e6;
}

/* one step at the current state: the captured step when there is one, else
 * capture it now (the capture runs the step) */
static int gen_step(uint32_t h) {
  if (hb_decoder_slot(h)) return thvm_hip_decoder_replay(h, 1);
  return thvm_hip_decoder_capture(h) ? 0 : -1;
}

/* Generation through the speculative step (reference run_spec /
 * serve_gen_spec, bench/dsv2_decode_bench.c:2629-2745, 2798-2860): the
 * prompt's first n_prompt-1 ids go through the one-row step, the last one
 * becomes the pending id the first speculative step verifies (P = n_prompt-1);
 * each step then commits 1..S ids (hist[P+1..]), read back once per burst.
 * A burst of n steps may advance the position by up to n*S, so it is sized
 * to keep every step's verify rows inside max_seq; when not even one fits,
 * the one-row step finishes the request. */
static int generate_spec(uint32_t h, const int32_t *prompt, uint32_t np, uint32_t max_new,
                         int32_t eos, int32_t *out, uint32_t *n_out, u32 S, u32 max_seq) {
  int rc = 0;
  for (u32 i = 0; i + 1 < np && !rc; i++) rc = thvm_hip_decoder_set_state(h, &prompt[i], i) || gen_step(h);
  if (!rc) rc = thvm_hip_decoder_set_state(h, &prompt[np - 1], np - 1);
  int32_t *hist = (int32_t *)malloc((u64)(max_seq + 1) * 4);
  if (!hist) { hb_set_error("decoder_generate: out of host memory"); return -1; }
  *n_out = 0;
  for (u32 k = 0; k < max_new; k++) out[k] = -1;
  u32 L = np;                      /* device length: P = L-1 is the pending position */
  while (!rc) {
    /* generated ids: hist[np .. L-1] (the new pending id included) */
    const u32 have = L - np;
    if (have > 0) {
      if (thvm_hip_decoder_read_tokens(h, hist, L)) { rc = -1; break; }
      int stop = 0;
      for (u32 k = *n_out; k < have && k < max_new; k++) {
        if (hist[np + k] == eos) { stop = 1; break; }
        out[k] = hist[np + k];
        *n_out = k + 1;
      }
      if (stop || *n_out >= max_new) break;
    }
    const u32 remaining = max_new - have;
    u32 burst = remaining < 8 ? remaining : 8;
    const u32 fit = (L - 1 + S <= max_seq) ? (max_seq - (L - 1)) / S : 0;
    if (burst > fit) burst = fit;
    if (burst == 0) {            /* no room for S verify rows: one-row steps */
      rc = gen_step(h);
    } else if (!hb_decoder_spec_slot(h)) {
      rc = thvm_hip_decoder_spec_capture(h) ? 0 : -1;   /* the capture runs step 1 */
    } else {
      rc = thvm_hip_decoder_spec_replay(h, burst);
    }
    if (!rc) {
      const u32 pos = thvm_hip_decoder_position(h);
      if (pos + 1 <= L) { hb_set_error("decoder_generate: the speculative step did not advance"); rc = -1; }
      L = pos + 1;
    }
  }
  free(hist);
  return rc;
}

THVM_API int thvm_hip_decoder_generate(uint32_t h, const int32_t *prompts, uint32_t n_prompt,
                                       uint32_t max_new, int32_t eos, int32_t *out,
                                       uint32_t *n_out) {
  u32 B = 0, S = 0, V = 0;
  if (hb_decoder_dims(h, &B, &S, &V)) return -1;
  if (!prompts || !out || !n_out) { hb_set_error("decoder_generate: null argument"); return -1; }
  if (n_prompt == 0) { hb_set_error("decoder_generate: empty prompt"); return -1; }
  if ((u64)n_prompt + max_new > S) {
    hb_set_error("decoder_generate: prompt %u + %u new ids exceed max_seq %u", n_prompt, max_new, S);
    return -1;
  }
  const u32 Ssp = hb_decoder_spec_rows(h);
  if (Ssp && B == 1 && n_prompt >= 2)
    return generate_spec(h, prompts, n_prompt, max_new, eos, out, n_out, Ssp, S);
  int32_t *tok = (int32_t *)malloc((u64)B * 4);
  int32_t *hist = (int32_t *)malloc((u64)B * (S + 1) * 4);
  if (!tok || !hist) { free(tok); free(hist); hb_set_error("decoder_generate: out of host memory"); return -1; }
  int rc = 0;
  /* prefill: position i consumes prompt id i (reference serve_prefill) */
  for (u32 i = 0; i < n_prompt && !rc; i++) {
    for (u32 b = 0; b < B; b++) tok[b] = prompts[(u64)b * n_prompt + i];
    rc = thvm_hip_decoder_set_state(h, tok, i) || gen_step(h);
  }
  for (u32 b = 0; b < B; b++) { n_out[b] = 0; for (u32 k = 0; k < max_new; k++) out[(u64)b * max_new + k] = -1; }
  /* generated id k sits at hist[n_prompt + k]; ids 1.. need one replay each */
  u32 have = max_new ? 1 : 0, done_rows = 0;
  uint8_t *done = (uint8_t *)calloc(B, 1);
  if (!done) rc = -1;
  while (!rc && have > 0) {
    if (thvm_hip_decoder_read_tokens(h, hist, n_prompt + have)) { rc = -1; break; }
    for (u32 b = 0; b < B; b++) {
      for (u32 k = n_out[b]; !done[b] && k < have; k++) {
        const int32_t id = hist[(u64)b * (n_prompt + have) + n_prompt + k];
        if (id == eos) { done[b] = 1; done_rows++; break; }
        out[(u64)b * max_new + k] = id;
        n_out[b] = k + 1;
      }
      if (!done[b] && n_out[b] == max_new) { done[b] = 1; done_rows++; }
    }
    if (done_rows == B || have == max_new) break;
    const u32 burst = max_new - have < 8 ? max_new - have : 8;
    if (thvm_hip_decoder_replay(h, burst)) { rc = -1; break; }
    have += burst;
  }
  free(done);
  free(tok);
  free(hist);
  return rc ? -1 : 0;
}

THVM_API int thvm_hip_decoder_serve(uint32_t h, int in_fd, int out_fd, int32_t eos,
                                    uint32_t default_max_new) {
  u32 B = 0, S = 0, V = 0;
  if (hb_decoder_dims(h, &B, &S, &V)) return -1;
  if (B != 1) { hb_set_error("decoder_serve: the serve loop decodes one sequence (batch 1), not %u", B); return -1; }
  int fi = dup(in_fd), fo = dup(out_fd);
  FILE *in = fi >= 0 ? fdopen(fi, "r") : NULL, *out = fo >= 0 ? fdopen(fo, "w") : NULL;
  if (!in || !out) {
    if (in) fclose(in); else if (fi >= 0) close(fi);
    if (out) fclose(out); else if (fo >= 0) close(fo);
    hb_set_error("decoder_serve: cannot open the request / response streams");
    return -1;
  }
  int32_t *prompt = (int32_t *)malloc((u64)S * 4), *gen = (int32_t *)malloc((u64)S * 4);
  char *line = NULL;
  size_t cap = 0;
  int rc = (prompt && gen) ? 0 : -1;
  if (!rc) { fputs("ready\n", out); fflush(out); }
  while (!rc) {
    ssize_t r = getline(&line, &cap, in);
    if (r < 0) break;                                   /* EOF: clean exit */
    u32 np = 0, max_new = default_max_new;
    char *bar = strchr(line, '|');
    if (bar) { max_new = (u32)strtoul(bar + 1, NULL, 10); *bar = 0; }
    const char *p = line;
    while (np < S && (*p == '-' || (*p >= '0' && *p <= '9'))) {
      char *end = NULL;
      long v = strtol(p, &end, 10);
      if (end == p) break;
      prompt[np++] = (int32_t)v;
      p = end;
      if (*p != ',') break;
      p++;
    }
    int bad = 0;
    for (u32 i = 0; i < np; i++) bad |= prompt[i] < 0 || (u32)prompt[i] >= V;
    long room = (long)S - (long)np;
    if (room < (long)max_new) max_new = room < 0 ? 0 : (u32)room;
    u32 n = 0;
    double t0 = now_ms();
    if (np > 0 && max_new > 0 && !bad)
      rc = thvm_hip_decoder_generate(h, prompt, np, max_new, eos, gen, &n);
    double ms = now_ms() - t0;
    fputs("ids: ", out);
    for (u32 i = 0; i < n; i++) fprintf(out, i ? ",%d" : "%d", gen[i]);
    fputs("\n", out);
    fflush(out);
    fprintf(stderr, "[serve] np=%u gen=%u %.1f ms (%.2f ms per position)%s\n", np, n, ms,
            np + n ? ms / (np + n) : 0.0, bad ? " [ids outside the vocabulary: refused]" : "");
  }
  free(line);
  free(prompt);
  free(gen);
  fclose(in);
  fclose(out);
  return rc;
}
