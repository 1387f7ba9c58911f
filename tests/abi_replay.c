/* Replays, from C, the call sequence of the Go binding go/hipnn/hipnn.go
 * (the reference side's loader for libdecide_hip.so), so that the binding's
 * use of the library is exercised without a Go toolchain:
 *
 *   Load     dlopen(path, RTLD_NOW | RTLD_GLOBAL) as purego.Dlopen does in
 *            internal/cuda/lib_unix.go:7-9, then one dlsym per symbol the
 *            binding registers (argv[2]: a file with one symbol per line); a
 *            failed dlopen or a missing symbol is ErrNoGPU, as Load says.
 *   New      dn_open(0) -> DN_NO_GPU is ErrNoGPU; dn_set_config,
 *            dn_upload_tensor per Tensors() entry, dn_weights_ready.
 *   Forward  the flattened batch through dn_forward.
 *   Evaluate the questions of one SystemOne call through dn_evaluate (one
 *            forward for all of them, as the wired decide.Local does).
 *   Free     dn_close.
 *
 * Without argv[3] the replay stops after dn_open (and dn_close when a device
 * was opened). argv[3] is a manifest written by tests/test_go_binding.py:
 *   config H I heads layers vocab eps half_window theta_g theta_l precision s_0 .. s_{layers-1}
 *   certify MARGIN         (dn_set_certify, before the tensors; NewWith's call)
 *   tensor NAME N          (N float32 values, in order, from argv[4])
 *   seq n has_opt nmask    then lines: ids, pos, [opt], mask positions
 *   question kind nopt n temperature   then a line of n token ids
 *   evaluate mask_id independent       (last: the questions through dn_evaluate)
 * Output lines: "ErrNoGPU (...)", "error <status> <message>", "ok <nlogits>"
 * followed by "logit <float32 bits in hex>" per logit; with `evaluate`,
 * "answers <nq>" followed by "answer <choice> <confidence> <value> <probs...>"
 * per question (doubles in %.17g). Exit status 0 unless the replay itself is
 * broken (bad manifest, unexpected status). */
#include <dlfcn.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

typedef int (*open_fn)(int, void **);
typedef void (*close_fn)(void *);
typedef const char *(*last_error_fn)(const void *);
typedef int (*set_config_fn)(void *, int, int, int, int, int, float, int, double, double, const uint8_t *, int);
typedef int (*upload_fn)(void *, const char *, const float *, int64_t);
typedef int (*ready_fn)(const void *);
typedef int (*forward_fn)(void *, int, const int32_t *, const int32_t *, const int32_t *, const int32_t *,
                          const int32_t *, const int32_t *, float *, int);
typedef int (*certify_fn)(void *, float);
typedef int (*evaluate_fn)(void *, int, const int32_t *, const int32_t *, const int32_t *, const int32_t *,
                           const double *, int32_t, int, double *, int32_t *, double *, double *);

enum { DN_OK = 0, DN_NO_GPU = 1 };

static void *need(void *h, const char *sym) {
  void *p = dlsym(h, sym);
  if (!p) {
    printf("ErrNoGPU (library is missing %s)\n", sym);
    exit(0);
  }
  return p;
}

static int read_ints(FILE *f, int32_t *dst, int n) {
  for (int i = 0; i < n; i++)
    if (fscanf(f, "%d", &dst[i]) != 1) return -1;
  return 0;
}

int main(int argc, char **argv) {
  if (argc < 3) {
    fprintf(stderr, "usage: abi_replay LIBRARY SYMBOLS [MANIFEST WEIGHTS]\n");
    return 2;
  }
  /* Load */
  void *h = dlopen(argv[1], RTLD_NOW | RTLD_GLOBAL);
  if (!h) {
    printf("ErrNoGPU (%s)\n", dlerror());
    return 0;
  }
  FILE *sf = fopen(argv[2], "r");
  if (!sf) return 2;
  char sym[256];
  int nsym = 0;
  while (fscanf(sf, "%255s", sym) == 1) {
    need(h, sym);
    nsym++;
  }
  fclose(sf);
  printf("resolved %d symbols\n", nsym);
  open_fn dn_open = (open_fn)need(h, "dn_open");
  close_fn dn_close = (close_fn)need(h, "dn_close");
  last_error_fn dn_last_error = (last_error_fn)need(h, "dn_last_error");
  set_config_fn dn_set_config = (set_config_fn)need(h, "dn_set_config");
  upload_fn dn_upload_tensor = (upload_fn)need(h, "dn_upload_tensor");
  ready_fn dn_weights_ready = (ready_fn)need(h, "dn_weights_ready");
  forward_fn dn_forward = (forward_fn)need(h, "dn_forward");
  certify_fn dn_set_certify = (certify_fn)need(h, "dn_set_certify");
  evaluate_fn dn_evaluate = (evaluate_fn)need(h, "dn_evaluate");

  /* New */
  void *ctx = NULL;
  int rc = dn_open(0, &ctx);
  if (rc == DN_NO_GPU) {
    printf("ErrNoGPU (%s)\n", dn_last_error(NULL));
    return 0;
  }
  if (rc != DN_OK) {
    printf("error %d %s\n", rc, dn_last_error(NULL));
    return 1;
  }
  if (argc < 5) {
    dn_close(ctx);
    printf("opened and closed\n");
    return 0;
  }
  FILE *mf = fopen(argv[3], "r"), *wf = fopen(argv[4], "rb");
  if (!mf || !wf) return 2;
  char word[256];
  int H, I, heads, layers, vocab, hw, prec;
  float eps;
  double tg, tl;
  if (fscanf(mf, "%255s %d %d %d %d %d %f %d %lf %lf %d", word, &H, &I, &heads, &layers, &vocab, &eps, &hw, &tg,
             &tl, &prec) != 11 || strcmp(word, "config"))
    return 2;
  uint8_t *sliding = calloc((size_t)layers + 1, 1);
  for (int l = 0; l < layers; l++) {
    int v;
    if (fscanf(mf, "%d", &v) != 1) return 2;
    sliding[l] = (uint8_t)v;
  }
  rc = dn_set_config(ctx, H, I, heads, layers, vocab, eps, hw, tg, tl, sliding, prec);
  if (rc != DN_OK) {
    printf("error %d %s\n", rc, dn_last_error(ctx));
    dn_close(ctx);
    return 0;
  }
  /* Tensors, then the batch. */
  int nseq = 0, T = 0, R = 0;
  int32_t *seq_len = NULL, *ids = NULL, *pos = NULL, *opt = NULL, *nmask = NULL, *mask = NULL;
  int any_opt = 0;
  int nq = 0, qtok = 0, do_eval = 0, eval_mask = 0, eval_ind = 0;
  int32_t *qkind = NULL, *qnopt = NULL, *qlen = NULL, *qids = NULL;
  double *qtemp = NULL;
  while (fscanf(mf, "%255s", word) == 1) {
    if (!strcmp(word, "certify")) {
      float margin;
      if (fscanf(mf, "%f", &margin) != 1) return 2;
      rc = dn_set_certify(ctx, margin);
      if (rc != DN_OK) {
        printf("error %d %s\n", rc, dn_last_error(ctx));
        dn_close(ctx);
        return 0;
      }
    } else if (!strcmp(word, "question")) {
      int kd, k, n;
      double t;
      if (fscanf(mf, "%d %d %d %lf", &kd, &k, &n, &t) != 4) return 2;
      qkind = realloc(qkind, sizeof(int32_t) * (nq + 1));
      qnopt = realloc(qnopt, sizeof(int32_t) * (nq + 1));
      qlen = realloc(qlen, sizeof(int32_t) * (nq + 1));
      qtemp = realloc(qtemp, sizeof(double) * (nq + 1));
      qids = realloc(qids, sizeof(int32_t) * (qtok + n + 1));
      if (read_ints(mf, qids + qtok, n)) return 2;
      qkind[nq] = kd, qnopt[nq] = k, qlen[nq] = n, qtemp[nq] = t;
      nq++;
      qtok += n;
    } else if (!strcmp(word, "evaluate")) {
      if (fscanf(mf, "%d %d", &eval_mask, &eval_ind) != 2) return 2;
      do_eval = 1;
    } else if (!strcmp(word, "tensor")) {
      char name[256];
      long long n;
      if (fscanf(mf, "%255s %lld", name, &n) != 2) return 2;
      float *buf = malloc(sizeof(float) * (size_t)n);
      if (fread(buf, sizeof(float), (size_t)n, wf) != (size_t)n) return 2;
      rc = dn_upload_tensor(ctx, name, buf, n);
      free(buf);
      if (rc != DN_OK) {
        printf("error %d %s\n", rc, dn_last_error(ctx));
        dn_close(ctx);
        return 0;
      }
    } else if (!strcmp(word, "seq")) {
      int n, has_opt, nm;
      if (fscanf(mf, "%d %d %d", &n, &has_opt, &nm) != 3) return 2;
      seq_len = realloc(seq_len, sizeof(int32_t) * (nseq + 1));
      nmask = realloc(nmask, sizeof(int32_t) * (nseq + 1));
      ids = realloc(ids, sizeof(int32_t) * (T + n));
      pos = realloc(pos, sizeof(int32_t) * (T + n));
      opt = realloc(opt, sizeof(int32_t) * (T + n));
      mask = realloc(mask, sizeof(int32_t) * (R + nm + 1));
      if (read_ints(mf, ids + T, n) || read_ints(mf, pos + T, n)) return 2;
      if (has_opt) {
        if (read_ints(mf, opt + T, n)) return 2;
        any_opt = 1;
      } else {
        for (int i = 0; i < n; i++) opt[T + i] = -1;  /* a nil OptID, as the binding passes it */
      }
      if (read_ints(mf, mask + R, nm)) return 2;
      seq_len[nseq] = n;
      nmask[nseq] = nm;
      nseq++;
      T += n;
      R += nm;
    } else {
      return 2;
    }
  }
  if (dn_weights_ready(ctx) != 1) {
    printf("error weights not ready\n");
    dn_close(ctx);
    return 1;
  }
  if (do_eval) {
    /* Evaluate: Model.Evaluate's single dn_evaluate call. */
    int nprob = 0;
    for (int q = 0; q < nq; q++) nprob += qnopt[q];
    double *probs = calloc((size_t)nprob + 1, sizeof(double)), *conf = calloc((size_t)nq + 1, sizeof(double));
    double *value = calloc((size_t)nq + 1, sizeof(double));
    int32_t *choice = calloc((size_t)nq + 1, sizeof(int32_t));
    rc = dn_evaluate(ctx, nq, qkind, qnopt, qlen, qids, qtemp, eval_mask, eval_ind, probs, choice, conf, value);
    if (rc != DN_OK) {
      printf("error %d %s\n", rc, dn_last_error(ctx));
    } else {
      printf("answers %d\n", nq);
      for (int q = 0, po = 0; q < nq; po += qnopt[q], q++) {
        printf("answer %d %.17g %.17g", choice[q], conf[q], value[q]);
        for (int i = 0; i < qnopt[q]; i++) printf(" %.17g", probs[po + i]);
        printf("\n");
      }
    }
    dn_close(ctx);
    free(probs), free(conf), free(value), free(choice);
    free(qkind), free(qnopt), free(qlen), free(qids), free(qtemp), free(sliding);
    return 0;
  }
  /* Forward */
  float *logits = calloc((size_t)R + 1, sizeof(float));
  rc = dn_forward(ctx, nseq, seq_len, ids, pos, any_opt ? opt : NULL, nmask, mask, logits, R);
  if (rc != DN_OK) {
    printf("error %d %s\n", rc, dn_last_error(ctx));
  } else {
    printf("ok %d\n", R);
    for (int r = 0; r < R; r++) {
      uint32_t bits;
      memcpy(&bits, &logits[r], 4);
      printf("logit %08x\n", bits);
    }
  }
  /* Free */
  dn_close(ctx);
  free(logits);
  free(seq_len), free(ids), free(pos), free(opt), free(nmask), free(mask), free(sliding);
  return 0;
}
