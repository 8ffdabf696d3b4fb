/*
 * CPU oracle for the Qwen3 batch-1 decode path -- TEST INFRASTRUCTURE ONLY.
 *
 * A plain-C restatement of metal_infrence_engine/src/cpu_inference.rs (the reference's CPU
 * engine), used by tests/ as the parity reference for the HIP engine and by bench.py as the
 * timed CPU baseline. The product (the HIP engine library) never links or calls this file.
 *
 * Build: oracle/Makefile (gcc -O2 -ffp-contract=off, no fast-math), so every f32 multiply and
 * add rounds separately, as in Rust. Each function cites the reference line it restates.
 */
#define _GNU_SOURCE
#include "oracle.h"

#include <errno.h>
#include <fcntl.h>
#include <math.h>
#include <pthread.h>
#include <sched.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

/* ------------------------------------------------------------------------------------------ */
/* minimal JSON reader (serde_json stand-in for the safetensors header and config.json)        */
/* ------------------------------------------------------------------------------------------ */

typedef enum { J_NULL, J_BOOL, J_NUM, J_STR, J_ARR, J_OBJ } jtype;

typedef struct jval {
  jtype t;
  int b;
  double num;
  int is_int;          /* number had no fraction/exponent */
  long long inum;      /* value if is_int and it fits */
  char* str;           /* J_STR */
  struct jval* items;  /* J_ARR / J_OBJ values */
  char** keys;         /* J_OBJ keys */
  size_t n;
} jval;

typedef struct {
  const char* s;
  size_t i, n;
  int err;
} jparser;

static void jfree(jval* v) {
  if (!v) return;
  if (v->t == J_STR) free(v->str);
  if (v->t == J_ARR || v->t == J_OBJ) {
    for (size_t i = 0; i < v->n; i++) {
      jfree(&v->items[i]);
      if (v->t == J_OBJ) free(v->keys[i]);
    }
    free(v->items);
    free(v->keys);
  }
}

static void jws(jparser* p) {
  while (p->i < p->n && (p->s[p->i] == ' ' || p->s[p->i] == '\t' || p->s[p->i] == '\n' || p->s[p->i] == '\r')) p->i++;
}

static int jparse_value(jparser* p, jval* out, int depth);

static int hexval(char c) {
  if (c >= '0' && c <= '9') return c - '0';
  if (c >= 'a' && c <= 'f') return c - 'a' + 10;
  if (c >= 'A' && c <= 'F') return c - 'A' + 10;
  return -1;
}

static char* jparse_string(jparser* p) {
  if (p->i >= p->n || p->s[p->i] != '"') { p->err = 1; return NULL; }
  p->i++;
  size_t cap = 16, len = 0;
  char* buf = malloc(cap);
  while (1) {
    if (p->i >= p->n) { p->err = 1; free(buf); return NULL; }
    unsigned char c = (unsigned char)p->s[p->i++];
    if (c == '"') break;
    if (c < 0x20) { p->err = 1; free(buf); return NULL; }
    unsigned cp = c;
    int raw = 1;
    if (c == '\\') {
      if (p->i >= p->n) { p->err = 1; free(buf); return NULL; }
      char e = p->s[p->i++];
      raw = 0;
      switch (e) {
        case '"': cp = '"'; break;
        case '\\': cp = '\\'; break;
        case '/': cp = '/'; break;
        case 'b': cp = '\b'; break;
        case 'f': cp = '\f'; break;
        case 'n': cp = '\n'; break;
        case 'r': cp = '\r'; break;
        case 't': cp = '\t'; break;
        case 'u': {
          if (p->i + 4 > p->n) { p->err = 1; free(buf); return NULL; }
          cp = 0;
          for (int k = 0; k < 4; k++) {
            int h = hexval(p->s[p->i++]);
            if (h < 0) { p->err = 1; free(buf); return NULL; }
            cp = cp * 16 + (unsigned)h;
          }
          if (cp >= 0xD800 && cp < 0xDC00) { /* surrogate pair */
            if (p->i + 6 > p->n || p->s[p->i] != '\\' || p->s[p->i + 1] != 'u') { p->err = 1; free(buf); return NULL; }
            p->i += 2;
            unsigned lo = 0;
            for (int k = 0; k < 4; k++) {
              int h = hexval(p->s[p->i++]);
              if (h < 0) { p->err = 1; free(buf); return NULL; }
              lo = lo * 16 + (unsigned)h;
            }
            if (lo < 0xDC00 || lo >= 0xE000) { p->err = 1; free(buf); return NULL; }
            cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
          } else if (cp >= 0xDC00 && cp < 0xE000) { p->err = 1; free(buf); return NULL; }
          break;
        }
        default: p->err = 1; free(buf); return NULL;
      }
    }
    char enc[4];
    int el;
    if (raw || cp < 0x80) { enc[0] = (char)cp; el = 1; }
    else if (cp < 0x800) { enc[0] = (char)(0xC0 | (cp >> 6)); enc[1] = (char)(0x80 | (cp & 0x3F)); el = 2; }
    else if (cp < 0x10000) { enc[0] = (char)(0xE0 | (cp >> 12)); enc[1] = (char)(0x80 | ((cp >> 6) & 0x3F)); enc[2] = (char)(0x80 | (cp & 0x3F)); el = 3; }
    else { enc[0] = (char)(0xF0 | (cp >> 18)); enc[1] = (char)(0x80 | ((cp >> 12) & 0x3F)); enc[2] = (char)(0x80 | ((cp >> 6) & 0x3F)); enc[3] = (char)(0x80 | (cp & 0x3F)); el = 4; }
    if (len + (size_t)el + 1 > cap) { cap = cap * 2 + (size_t)el; buf = realloc(buf, cap); }
    memcpy(buf + len, enc, (size_t)el);
    len += (size_t)el;
  }
  buf[len] = 0;
  return buf;
}

static int jparse_value(jparser* p, jval* out, int depth) {
  memset(out, 0, sizeof(*out));
  if (depth > 64) { p->err = 1; return -1; }
  jws(p);
  if (p->i >= p->n) { p->err = 1; return -1; }
  char c = p->s[p->i];
  if (c == '{' || c == '[') {
    int obj = c == '{';
    out->t = obj ? J_OBJ : J_ARR;
    p->i++;
    size_t cap = 0;
    jws(p);
    if (p->i < p->n && p->s[p->i] == (obj ? '}' : ']')) { p->i++; return 0; }
    while (1) {
      jws(p);
      char* key = NULL;
      if (obj) {
        key = jparse_string(p);
        if (!key) return -1;
        jws(p);
        if (p->i >= p->n || p->s[p->i] != ':') { free(key); p->err = 1; return -1; }
        p->i++;
      }
      if (out->n == cap) {
        cap = cap ? cap * 2 : 8;
        jval* items = realloc(out->items, cap * sizeof(jval));
        if (items) out->items = items;
        char** keys = obj ? realloc(out->keys, cap * sizeof(char*)) : NULL;
        if (keys) out->keys = keys;
        if (!items || (obj && !keys)) { free(key); p->err = 1; return -1; }
      }
      /* a failed child is freed here; the caller frees this value's first n items */
      if (jparse_value(p, &out->items[out->n], depth + 1) != 0) {
        jfree(&out->items[out->n]);
        free(key);
        return -1;
      }
      if (obj) out->keys[out->n] = key;
      out->n++;
      jws(p);
      if (p->i >= p->n) { p->err = 1; return -1; }
      if (p->s[p->i] == ',') { p->i++; continue; }
      if (p->s[p->i] == (obj ? '}' : ']')) { p->i++; return 0; }
      p->err = 1;
      return -1;
    }
  }
  if (c == '"') {
    out->t = J_STR;
    out->str = jparse_string(p);
    return out->str ? 0 : -1;
  }
  if (p->n - p->i >= 4 && memcmp(p->s + p->i, "true", 4) == 0) { out->t = J_BOOL; out->b = 1; p->i += 4; return 0; }
  if (p->n - p->i >= 5 && memcmp(p->s + p->i, "false", 5) == 0) { out->t = J_BOOL; out->b = 0; p->i += 5; return 0; }
  if (p->n - p->i >= 4 && memcmp(p->s + p->i, "null", 4) == 0) { out->t = J_NULL; p->i += 4; return 0; }
  if (c == '-' || (c >= '0' && c <= '9')) {
    size_t st = p->i;
    int is_int = 1;
    if (p->s[p->i] == '-') p->i++;
    if (p->i >= p->n || !(p->s[p->i] >= '0' && p->s[p->i] <= '9')) { p->err = 1; return -1; }
    while (p->i < p->n && p->s[p->i] >= '0' && p->s[p->i] <= '9') p->i++;
    if (p->i < p->n && p->s[p->i] == '.') {
      is_int = 0;
      p->i++;
      if (p->i >= p->n || !(p->s[p->i] >= '0' && p->s[p->i] <= '9')) { p->err = 1; return -1; }
      while (p->i < p->n && p->s[p->i] >= '0' && p->s[p->i] <= '9') p->i++;
    }
    if (p->i < p->n && (p->s[p->i] == 'e' || p->s[p->i] == 'E')) {
      is_int = 0;
      p->i++;
      if (p->i < p->n && (p->s[p->i] == '+' || p->s[p->i] == '-')) p->i++;
      if (p->i >= p->n || !(p->s[p->i] >= '0' && p->s[p->i] <= '9')) { p->err = 1; return -1; }
      while (p->i < p->n && p->s[p->i] >= '0' && p->s[p->i] <= '9') p->i++;
    }
    char tmp[64];
    size_t l = p->i - st;
    if (l >= sizeof(tmp)) { p->err = 1; return -1; }
    memcpy(tmp, p->s + st, l);
    tmp[l] = 0;
    out->t = J_NUM;
    out->num = strtod(tmp, NULL);
    out->is_int = 0;
    if (is_int) {
      errno = 0;
      long long v = strtoll(tmp, NULL, 10);
      if (errno == 0) { out->is_int = 1; out->inum = v; }
    }
    return 0;
  }
  p->err = 1;
  return -1;
}

/* On failure *out is freed and left as an empty null value. */
static int jparse(const char* s, size_t n, jval* out) {
  jparser p = {s, 0, n, 0};
  int rc = jparse_value(&p, out, 0);
  if (rc == 0) {
    jws(&p);
    if (p.i != p.n) rc = -1;
  }
  if (rc != 0) {
    jfree(out);
    memset(out, 0, sizeof(*out));
  }
  return rc;
}

static const jval* jget(const jval* obj, const char* key) {
  if (!obj || obj->t != J_OBJ) return NULL;
  const jval* found = NULL;
  for (size_t i = 0; i < obj->n; i++)
    if (strcmp(obj->keys[i], key) == 0) found = &obj->items[i]; /* last duplicate wins, as a map insert */
  return found;
}

/* ------------------------------------------------------------------------------------------ */
/* model                                                                                        */
/* ------------------------------------------------------------------------------------------ */

typedef struct {
  char* name;
  char* dtype;
  int64_t* shape;
  size_t ndim;
  int64_t off0, off1;
} or_tensor;

struct or_model {
  void* map;
  size_t map_len;
  const uint8_t* raw;       /* data section, cpu_inference.rs:74 */
  or_tensor* tensors;
  size_t ntensors;
  or_config cfg;
};

struct or_kvcache {
  size_t layers, kv_dim, len, cap;   /* len = cached positions */
  int bf16;                          /* append K/V rounded to bf16 (or_kv_new_bf16) */
  float** k;
  float** v;
};

static void seterr(char* err, size_t errlen, const char* fmt, ...) {
  if (!err || !errlen) return;
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(err, errlen, fmt, ap);
  va_end(ap);
}

void or_free_model(or_model* m) {
  if (!m) return;
  for (size_t i = 0; i < m->ntensors; i++) {
    free(m->tensors[i].name);
    free(m->tensors[i].dtype);
    free(m->tensors[i].shape);
  }
  free(m->tensors);
  if (m->map) munmap(m->map, m->map_len);
  free(m);
}

/* serde: usize from a non-negative JSON integer */
static int get_usize(const jval* o, const char* k, uint64_t* out) {
  const jval* v = jget(o, k);
  if (!v || v->t != J_NUM || !v->is_int || v->inum < 0) return -1;
  *out = (uint64_t)v->inum;
  return 0;
}
/* serde: f32 from any JSON number (parsed as f64, then `as f32`) */
static int get_f32(const jval* o, const char* k, float* out) {
  const jval* v = jget(o, k);
  if (!v || v->t != J_NUM) return -1;
  *out = (float)v->num;
  return 0;
}

static int read_config(const char* model_path, or_config* cfg, char* err, size_t errlen, int* status) {
  /* cpu_inference.rs:80-81: config.json next to the weights file */
  char path[4096];
  const char* slash = strrchr(model_path, '/');
  if (slash) {
    size_t dl = (size_t)(slash - model_path) + 1;
    if (dl + 12 >= sizeof(path)) { *status = OR_ERR_IO; seterr(err, errlen, "path too long"); return -1; }
    memcpy(path, model_path, dl);
    strcpy(path + dl, "config.json");
  } else {
    strcpy(path, "config.json");
  }
  FILE* f = fopen(path, "rb");
  if (!f) { *status = OR_ERR_IO; seterr(err, errlen, "cannot open %s: %s", path, strerror(errno)); return -1; }
  fseek(f, 0, SEEK_END);
  long n = ftell(f);
  fseek(f, 0, SEEK_SET);
  char* buf = malloc((size_t)n + 1);
  size_t got = fread(buf, 1, (size_t)n, f);
  fclose(f);
  jval root;
  if (got != (size_t)n || jparse(buf, (size_t)n, &root) != 0) {
    free(buf);
    *status = OR_ERR_FORMAT;
    seterr(err, errlen, "config.json is not valid JSON");
    return -1;
  }
  free(buf);
  uint64_t eos = 0;
  int bad = root.t != J_OBJ;
  bad |= get_usize(&root, "hidden_size", &cfg->hidden_size);
  bad |= get_usize(&root, "intermediate_size", &cfg->intermediate_size);
  bad |= get_usize(&root, "num_hidden_layers", &cfg->num_hidden_layers);
  bad |= get_usize(&root, "num_attention_heads", &cfg->num_attention_heads);
  bad |= get_usize(&root, "num_key_value_heads", &cfg->num_key_value_heads);
  bad |= get_usize(&root, "head_dim", &cfg->head_dim);
  bad |= get_usize(&root, "vocab_size", &cfg->vocab_size);
  bad |= get_f32(&root, "rms_norm_eps", &cfg->rms_norm_eps);
  bad |= get_f32(&root, "rope_theta", &cfg->rope_theta);
  bad |= get_usize(&root, "eos_token_id", &eos);
  jfree(&root);
  if (bad || eos > 0xFFFFFFFFull) {
    *status = OR_ERR_FORMAT;
    seterr(err, errlen, "config.json is missing a field or has the wrong type");
    return -1;
  }
  cfg->eos_token_id = (uint32_t)eos;
  return 0;
}

or_model* or_load_model(const char* path, int* status, char* err, size_t errlen) {
  int st_dummy;
  if (!status) status = &st_dummy;
  *status = OR_OK;
  /* cpu_inference.rs:60-61 */
  int fd = open(path, O_RDONLY);
  if (fd < 0) { *status = OR_ERR_IO; seterr(err, errlen, "cannot open %s: %s", path, strerror(errno)); return NULL; }
  struct stat sb;
  if (fstat(fd, &sb) != 0) { close(fd); *status = OR_ERR_IO; seterr(err, errlen, "stat failed"); return NULL; }
  size_t len = (size_t)sb.st_size;
  void* map = len ? mmap(NULL, len, PROT_READ, MAP_PRIVATE, fd, 0) : NULL;
  close(fd);
  if (len && map == MAP_FAILED) { *status = OR_ERR_IO; seterr(err, errlen, "mmap failed"); return NULL; }
  or_model* m = calloc(1, sizeof(*m));
  m->map = len ? map : NULL;
  m->map_len = len;
  const uint8_t* b = (const uint8_t*)map;
  /* cpu_inference.rs:62-64: u64 LE header length, then UTF-8 JSON */
  if (len < 8) { *status = OR_ERR_FORMAT; seterr(err, errlen, "file shorter than the 8-byte header length"); or_free_model(m); return NULL; }
  uint64_t hl = 0;
  for (int i = 7; i >= 0; i--) hl = (hl << 8) | b[i];
  if (hl > len - 8) { *status = OR_ERR_FORMAT; seterr(err, errlen, "header length %llu exceeds file size", (unsigned long long)hl); or_free_model(m); return NULL; }
  /* cpu_inference.rs:65-73: parse; skip __metadata__; every other key is a Tensor */
  jval root;
  if (jparse((const char*)b + 8, (size_t)hl, &root) != 0 || root.t != J_OBJ) {
    if (root.t == J_OBJ) jfree(&root);
    *status = OR_ERR_FORMAT;
    seterr(err, errlen, "safetensors header is not a JSON object");
    or_free_model(m);
    return NULL;
  }
  m->tensors = calloc(root.n ? root.n : 1, sizeof(or_tensor));
  for (size_t i = 0; i < root.n; i++) {
    if (strcmp(root.keys[i], "__metadata__") == 0) continue;
    const jval* tv = &root.items[i];
    const jval* dt = jget(tv, "dtype");
    const jval* sh = jget(tv, "shape");
    const jval* of = jget(tv, "data_offsets");
    int bad = !dt || dt->t != J_STR || !sh || sh->t != J_ARR || !of || of->t != J_ARR || of->n != 2;
    if (!bad) {
      for (size_t k = 0; k < sh->n; k++)
        if (sh->items[k].t != J_NUM || !sh->items[k].is_int || sh->items[k].inum < INT32_MIN || sh->items[k].inum > INT32_MAX) bad = 1;
      for (size_t k = 0; k < 2; k++)
        if (of->items[k].t != J_NUM || !of->items[k].is_int || of->items[k].inum < INT32_MIN || of->items[k].inum > INT32_MAX) bad = 1;
    }
    if (bad) {
      seterr(err, errlen, "tensor %s: bad header entry", root.keys[i]);
      jfree(&root);
      *status = OR_ERR_FORMAT;
      or_free_model(m);
      return NULL;
    }
    or_tensor* t = &m->tensors[m->ntensors++];
    t->name = strdup(root.keys[i]);
    t->dtype = strdup(dt->str);
    t->ndim = sh->n;
    t->shape = calloc(sh->n ? sh->n : 1, sizeof(int64_t));
    for (size_t k = 0; k < sh->n; k++) t->shape[k] = sh->items[k].inum;
    t->off0 = of->items[0].inum;
    t->off1 = of->items[1].inum;
  }
  jfree(&root);
  /* cpu_inference.rs:74-76 */
  m->raw = b + 8 + hl;
  if (((uintptr_t)m->raw) % 2 != 0) { *status = OR_ERR_FORMAT; seterr(err, errlen, "safetensors data section is not 2-byte aligned"); or_free_model(m); return NULL; }
  if (read_config(path, &m->cfg, err, errlen, status) != 0) { or_free_model(m); return NULL; }
  return m;
}

void or_get_config(const or_model* m, or_config* out) { *out = m->cfg; }
size_t or_num_tensors(const or_model* m) { return m->ntensors; }
int or_tensor_info(const or_model* m, size_t i, const char** name, const char** dtype, int64_t* off0, int64_t* off1) {
  if (i >= m->ntensors) return OR_ERR_ARG;
  *name = m->tensors[i].name;
  *dtype = m->tensors[i].dtype;
  *off0 = m->tensors[i].off0;
  *off1 = m->tensors[i].off1;
  return OR_OK;
}

/* cpu_inference.rs:86-96 Model::weight: bf16 view of a tensor, with its checks */
static const uint16_t* weight(const or_model* m, const char* name, size_t* numel_out) {
  const or_tensor* t = NULL;
  for (size_t i = 0; i < m->ntensors; i++)
    if (strcmp(m->tensors[i].name, name) == 0) t = &m->tensors[i];
  if (!t) return NULL;                               /* panic "missing tensor" */
  if (strcmp(t->dtype, "BF16") != 0) return NULL;    /* panic "only BF16" */
  if (t->off0 < 0 || t->off1 < t->off0) return NULL;
  size_t numel = 1;
  for (size_t k = 0; k < t->ndim; k++) numel *= (size_t)t->shape[k];
  if ((size_t)(t->off1 - t->off0) / 2 != numel) return NULL; /* assert_eq numel */
  if ((size_t)t->off1 > m->map_len - (size_t)(m->raw - (const uint8_t*)m->map)) return NULL;
  if (numel_out) *numel_out = numel;
  return (const uint16_t*)(m->raw + t->off0);
}

/* ------------------------------------------------------------------------------------------ */
/* math helpers: cpu_inference.rs:182-257                                                       */
/* ------------------------------------------------------------------------------------------ */

/* :182-183 */
float or_bf16_to_f32(uint16_t x) {
  uint32_t u = (uint32_t)x << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

/* Rust's `impl Sum for f32` folds from -0.0 in order */
static inline float sum_f32(const float* a, size_t n) {
  float s = -0.0f;
  for (size_t i = 0; i < n; i++) s = s + a[i];
  return s;
}

/* :185 dot = a.zip(b).map(x*y).sum() */
float or_dot(const float* a, const float* b, size_t n) {
  float s = -0.0f;
  for (size_t i = 0; i < n; i++) s = s + a[i] * b[i];
  return s;
}

/* :187 */
float or_silu(float x) { return x / (1.0f + expf(-x)); }

/* :189-194 */
void or_rmsnorm(float* out, const float* x, const uint16_t* w, size_t n, float eps) {
  float ss = -0.0f;
  for (size_t i = 0; i < n; i++) ss = ss + x[i] * x[i];
  float ms = ss / (float)n;
  float s = 1.0f / sqrtf(ms + eps);
  for (size_t i = 0; i < n; i++) out[i] = x[i] * s * or_bf16_to_f32(w[i]);
}

/* :196-201 */
void or_rmsnorm_inplace(float* x, const uint16_t* w, size_t n, float eps) {
  float ss = -0.0f;
  for (size_t i = 0; i < n; i++) ss = ss + x[i] * x[i];
  float ms = ss / (float)n;
  float s = 1.0f / sqrtf(ms + eps);
  for (size_t i = 0; i < n; i++) x[i] = x[i] * s * or_bf16_to_f32(w[i]);
}

/* :203-215 rotate-half RoPE; freq = theta.powf(-2.0 * i as f32 / len as f32) */
void or_rope(float* x, size_t n, size_t pos, float theta) {
  size_t half = n / 2;
  for (size_t i = 0; i < half; i++) {
    float freq = powf(theta, -2.0f * (float)i / (float)n);
    float ang = (float)pos * freq;
    float sn = sinf(ang), cs = cosf(ang);
    float a = x[i], b = x[i + half];
    x[i] = a * cs - b * sn;
    x[i + half] = b * cs + a * sn;
  }
}

/* metal_inference.rs:140-154: the same expressions as rope(), tabulated per position */
void or_rope_table(float* out, size_t max_seq, size_t head_dim, float theta) {
  size_t half = head_dim / 2;
  for (size_t pos = 0; pos < max_seq; pos++)
    for (size_t i = 0; i < half; i++) {
      float freq = powf(theta, -2.0f * (float)i / (float)head_dim);
      float ang = (float)pos * freq;
      out[(pos * half + i) * 2 + 0] = cosf(ang);
      out[(pos * half + i) * 2 + 1] = sinf(ang);
    }
}

/* :217-223 */
void or_softmax(float* x, size_t n) {
  float mx = -INFINITY;
  for (size_t i = 0; i < n; i++) mx = fmaxf(mx, x[i]); /* f32::max ignores NaN, like fmaxf */
  float sum = 0.0f;
  for (size_t i = 0; i < n; i++) { x[i] = expf(x[i] - mx); sum += x[i]; }
  for (size_t i = 0; i < n; i++) x[i] /= sum;
}

/* :243-257: 8 independent accumulators over chunks of 8, sequential sum, then the remainder */
float or_dot_bf16(const uint16_t* w, const float* x, size_t n) {
  float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  size_t chunks = n / 8;
  for (size_t c = 0; c < chunks; c++)
    for (int i = 0; i < 8; i++) acc[i] += or_bf16_to_f32(w[c * 8 + (size_t)i]) * x[c * 8 + (size_t)i];
  float s = sum_f32(acc, 8);
  for (size_t i = chunks * 8; i < n; i++) s += or_bf16_to_f32(w[i]) * x[i];
  return s;
}

/* ---- :225-241 matvec, rows chunked across available_parallelism() threads spawned per call ---- */

static int g_threads = 0;

static int detect_threads(void) {
  const char* e = getenv("QE_ORACLE_THREADS");
  if (e && atoi(e) > 0) return atoi(e);
  cpu_set_t set;
  if (sched_getaffinity(0, sizeof(set), &set) == 0) {
    int n = CPU_COUNT(&set);
    if (n > 0) return n;
  }
  long n = sysconf(_SC_NPROCESSORS_ONLN);
  return n > 0 ? (int)n : 1;
}

void or_set_threads(int n) { g_threads = n > 0 ? n : detect_threads(); if (g_threads > 1024) g_threads = 1024; }
int or_get_threads(void) {
  if (g_threads <= 0) g_threads = detect_threads();
  if (g_threads > 1024) g_threads = 1024;
  return g_threads;
}

typedef struct {
  float* out;
  const uint16_t* w;
  const float* x;
  size_t rows, cols;
} mv_job;

static void* mv_worker(void* arg) {
  mv_job* j = (mv_job*)arg;
  for (size_t r = 0; r < j->rows; r++) j->out[r] = or_dot_bf16(j->w + r * j->cols, j->x, j->cols);
  return NULL;
}

void or_matvec(float* out, const uint16_t* w, const float* x, size_t rows, size_t cols) {
  int threads = or_get_threads();
  size_t rows_per = (rows + (size_t)threads - 1) / (size_t)threads; /* div_ceil */
  if (rows_per == 0) return;
  size_t nchunks = (rows + rows_per - 1) / rows_per;              /* out.chunks_mut(rows_per) */
  pthread_t tids[1024];
  mv_job jobs[1024];
  size_t spawned = 0;
  for (size_t c = 0; c < nchunks; c++) {
    size_t r0 = c * rows_per;
    size_t nr = rows - r0 < rows_per ? rows - r0 : rows_per;
    jobs[c] = (mv_job){out + r0, w + r0 * cols, x, nr, cols};
    if (nchunks == 1 || pthread_create(&tids[c], NULL, mv_worker, &jobs[c]) != 0) {
      mv_worker(&jobs[c]);   /* single chunk (or spawn failure): run inline; results are identical */
      tids[c] = 0;
    } else {
      spawned++;
    }
  }
  for (size_t c = 0; c < nchunks; c++)
    if (tids[c]) pthread_join(tids[c], NULL);
  (void)spawned;
}

/* ------------------------------------------------------------------------------------------ */
/* KV cache: cpu_inference.rs:44-55 (per layer Vec<f32>, appended per position)                */
/* ------------------------------------------------------------------------------------------ */

or_kvcache* or_kv_new(const or_model* m) {
  or_kvcache* c = calloc(1, sizeof(*c));
  c->bf16 = 0;
  c->layers = m->cfg.num_hidden_layers;
  c->kv_dim = m->cfg.num_key_value_heads * m->cfg.head_dim;
  c->k = calloc(c->layers ? c->layers : 1, sizeof(float*));
  c->v = calloc(c->layers ? c->layers : 1, sizeof(float*));
  return c;
}

/* A cache that keeps each appended K/V element rounded to bf16 (round to nearest, ties to even)
 * and attends with the rounded values. The reference has no such cache on its main branch
 * (README.md:23,90 reports one only as an experiment); this mode states that rounding exactly so
 * a bf16 device cache has something independent to be compared with. */
or_kvcache* or_kv_new_bf16(const or_model* m) {
  or_kvcache* c = or_kv_new(m);
  c->bf16 = 1;
  return c;
}

/* f32 -> nearest bf16 value (ties to even), returned widened back to f32. NaN stays NaN (quiet),
 * values past the largest bf16 round to infinity as IEEE rounding does. */
float or_round_bf16(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) u = (u | 0x00400000u) & 0xFFFF0000u;
  else u = (u + 0x7FFFu + ((u >> 16) & 1u)) & 0xFFFF0000u;
  float r;
  memcpy(&r, &u, 4);
  return r;
}

void or_kv_free(or_kvcache* c) {
  if (!c) return;
  for (size_t l = 0; l < c->layers; l++) { free(c->k[l]); free(c->v[l]); }
  free(c->k);
  free(c->v);
  free(c);
}

size_t or_kv_len(const or_kvcache* c) { return c->len; }

static void kv_reserve(or_kvcache* c, size_t npos) {
  if (npos <= c->cap) return;
  size_t nc = c->cap ? c->cap : 64;
  while (nc < npos) nc *= 2;
  for (size_t l = 0; l < c->layers; l++) {
    c->k[l] = realloc(c->k[l], nc * c->kv_dim * sizeof(float));
    c->v[l] = realloc(c->v[l], nc * c->kv_dim * sizeof(float));
  }
  c->cap = nc;
}

/* cpu_inference.rs:144-162, one layer, for all heads */
void or_attention(const float* q, const float* kc, const float* vc, size_t n_pos, size_t n_heads,
                  size_t n_kv_heads, size_t hd, float* att) {
  size_t kv_dim = n_kv_heads * hd;
  size_t group = n_heads / n_kv_heads;
  float scale = 1.0f / sqrtf((float)hd);
  float* scores = malloc((n_pos ? n_pos : 1) * sizeof(float));
  for (size_t h = 0; h < n_heads; h++) {
    const float* qh = q + h * hd;
    size_t kv_off = (h / group) * hd;
    for (size_t t = 0; t < n_pos; t++) scores[t] = or_dot(qh, kc + t * kv_dim + kv_off, hd) * scale;
    or_softmax(scores, n_pos);
    float* out = att + h * hd;
    for (size_t i = 0; i < hd; i++) out[i] = 0.0f;
    for (size_t t = 0; t < n_pos; t++) {
      const float* vt = vc + t * kv_dim + kv_off;
      for (size_t i = 0; i < hd; i++) out[i] += scores[t] * vt[i];
    }
  }
  free(scores);
}

/* ------------------------------------------------------------------------------------------ */
/* forward: cpu_inference.rs:98-179                                                              */
/* ------------------------------------------------------------------------------------------ */

#define W(name) do { \
    snprintf(nm, sizeof(nm), "model.layers.%zu.%s", l, name); \
  } while (0)

int or_forward(const or_model* m, uint32_t token, size_t pos, or_kvcache* cache, float* logits) {
  const or_config* c = &m->cfg;
  size_t hd = c->head_dim;
  size_t q_dim = c->num_attention_heads * hd;
  size_t kv_dim = c->num_key_value_heads * hd;
  float eps = c->rms_norm_eps;
  size_t H = c->hidden_size, I = c->intermediate_size;
  if (c->num_key_value_heads == 0 || c->num_attention_heads % c->num_key_value_heads) return OR_ERR_ARG;
  /* the reference appends at the end and attends 0..=pos, so pos must equal the cached length */
  if (pos != cache->len) return OR_ERR_POS;

  size_t n_embed;
  const uint16_t* embed = weight(m, "model.embed_tokens.weight", &n_embed);
  if (!embed) return OR_ERR_TENSOR;
  if ((size_t)token * H + H > n_embed) return OR_ERR_ARG;

  float* x = malloc(H * sizeof(float));
  float* xn = malloc(H * sizeof(float));
  float* q = malloc(q_dim * sizeof(float));
  float* k = malloc(kv_dim * sizeof(float));
  float* v = malloc(kv_dim * sizeof(float));
  float* att = malloc(q_dim * sizeof(float));
  float* proj = malloc(H * sizeof(float));
  float* gate = malloc(I * sizeof(float));
  float* up = malloc(I * sizeof(float));
  int rc = OR_OK;
  char nm[256];

  for (size_t i = 0; i < H; i++) x[i] = or_bf16_to_f32(embed[(size_t)token * H + i]);
  kv_reserve(cache, pos + 1);

  for (size_t l = 0; l < c->num_hidden_layers && rc == OR_OK; l++) {
    size_t n;
    const uint16_t *w_in, *wq, *wk, *wv, *wqn, *wkn, *wo, *w_post, *wg, *wu, *wd;
    W("input_layernorm.weight"); w_in = weight(m, nm, &n); if (!w_in || n != H) { rc = OR_ERR_TENSOR; break; }
    W("self_attn.q_proj.weight"); wq = weight(m, nm, &n); if (!wq || n != q_dim * H) { rc = OR_ERR_TENSOR; break; }
    W("self_attn.k_proj.weight"); wk = weight(m, nm, &n); if (!wk || n != kv_dim * H) { rc = OR_ERR_TENSOR; break; }
    W("self_attn.v_proj.weight"); wv = weight(m, nm, &n); if (!wv || n != kv_dim * H) { rc = OR_ERR_TENSOR; break; }
    W("self_attn.q_norm.weight"); wqn = weight(m, nm, &n); if (!wqn || n != hd) { rc = OR_ERR_TENSOR; break; }
    W("self_attn.k_norm.weight"); wkn = weight(m, nm, &n); if (!wkn || n != hd) { rc = OR_ERR_TENSOR; break; }
    W("self_attn.o_proj.weight"); wo = weight(m, nm, &n); if (!wo || n != H * q_dim) { rc = OR_ERR_TENSOR; break; }
    W("post_attention_layernorm.weight"); w_post = weight(m, nm, &n); if (!w_post || n != H) { rc = OR_ERR_TENSOR; break; }
    W("mlp.gate_proj.weight"); wg = weight(m, nm, &n); if (!wg || n != I * H) { rc = OR_ERR_TENSOR; break; }
    W("mlp.up_proj.weight"); wu = weight(m, nm, &n); if (!wu || n != I * H) { rc = OR_ERR_TENSOR; break; }
    W("mlp.down_proj.weight"); wd = weight(m, nm, &n); if (!wd || n != H * I) { rc = OR_ERR_TENSOR; break; }

    /* attention: :129-132 */
    or_rmsnorm(xn, x, w_in, H, eps);
    or_matvec(q, wq, xn, q_dim, H);
    or_matvec(k, wk, xn, kv_dim, H);
    or_matvec(v, wv, xn, kv_dim, H);
    /* :134-138 per-head q/k rmsnorm, then rope */
    for (size_t h = 0; h < c->num_attention_heads; h++) { or_rmsnorm_inplace(q + h * hd, wqn, hd, eps); or_rope(q + h * hd, hd, pos, c->rope_theta); }
    for (size_t h = 0; h < c->num_key_value_heads; h++) { or_rmsnorm_inplace(k + h * hd, wkn, hd, eps); or_rope(k + h * hd, hd, pos, c->rope_theta); }
    /* :140-142 append (a bf16 cache stores, and later attends with, the rounded values) */
    if (cache->bf16)
      for (size_t i = 0; i < kv_dim; i++) { k[i] = or_round_bf16(k[i]); v[i] = or_round_bf16(v[i]); }
    memcpy(cache->k[l] + pos * kv_dim, k, kv_dim * sizeof(float));
    memcpy(cache->v[l] + pos * kv_dim, v, kv_dim * sizeof(float));
    /* :144-162 */
    or_attention(q, cache->k[l], cache->v[l], pos + 1, c->num_attention_heads, c->num_key_value_heads, hd, att);
    /* :163-164 */
    or_matvec(proj, wo, att, H, q_dim);
    for (size_t i = 0; i < H; i++) x[i] += proj[i];
    /* :166-172 swiglu */
    or_rmsnorm(xn, x, w_post, H, eps);
    or_matvec(gate, wg, xn, I, H);
    or_matvec(up, wu, xn, I, H);
    for (size_t i = 0; i < I; i++) gate[i] = or_silu(gate[i]) * up[i];
    or_matvec(proj, wd, gate, H, I);
    for (size_t i = 0; i < H; i++) x[i] += proj[i];
  }
  if (rc == OR_OK) {
    size_t n;
    /* :175-178 */
    const uint16_t* wn = weight(m, "model.norm.weight", &n);
    const uint16_t* wl = weight(m, "lm_head.weight", NULL);
    if (!wn || n != H || !wl) rc = OR_ERR_TENSOR;
    else {
      weight(m, "lm_head.weight", &n);
      if (n != c->vocab_size * H) rc = OR_ERR_TENSOR;
      else {
        or_rmsnorm(xn, x, wn, H, eps);
        or_matvec(logits, wl, xn, c->vocab_size, H);
        cache->len = pos + 1;
      }
    }
  }
  free(x); free(xn); free(q); free(k); free(v); free(att); free(proj); free(gate); free(up);
  return rc;
}

/* main.rs:37-42 */
uint32_t or_argmax(const float* x, size_t n) {
  size_t best = 0;
  for (size_t i = 1; i < n; i++)
    if (x[i] > x[best]) best = i;
  return (uint32_t)best;
}

/* bench.rs:106-116: every tensor except the embedding table, plus one embedding row */
uint64_t or_weight_bytes_per_token(const or_model* m) {
  uint64_t bytes = 0;
  for (size_t i = 0; i < m->ntensors; i++) {
    if (strcmp(m->tensors[i].name, "model.embed_tokens.weight") == 0) continue;
    bytes += (uint64_t)(m->tensors[i].off1 - m->tensors[i].off0);
  }
  return bytes + m->cfg.hidden_size * 2;
}

/* bench.rs:118-119 */
uint64_t or_kv_bytes_at(const or_config* c, uint64_t pos) {
  return 2 * c->num_hidden_layers * (pos + 1) * c->num_key_value_heads * c->head_dim * 4;
}
