#include "core/safetensors.h"
#include "core/json.h"
#include "core/devmem.h"
#include <dirent.h>
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

struct st_file {
    int fd;
    void *map;
    size_t size;
    js_doc *header; /* owns the tensor name strings */
};

static void st_file_close(st_file *f) {
    if (!f)
        return;
    js_free(f->header);
    if (f->map && f->map != MAP_FAILED)
        munmap(f->map, f->size);
    if (f->fd >= 0)
        close(f->fd);
    free(f);
}

/* FNV-1a over the name bytes. */
static uint32_t name_hash(const char *s) {
    uint32_t h = 2166136261u;
    for (; *s; s++)
        h = (h ^ (uint8_t)*s) * 16777619u;
    return h;
}

static st_dtype parse_dtype(const char *s) {
    if (strcmp(s, "BF16") == 0)
        return ST_BF16;
    if (strcmp(s, "F16") == 0)
        return ST_F16;
    if (strcmp(s, "F32") == 0)
        return ST_F32;
    return ST_OTHER;
}

static size_t dtype_size(st_dtype d) { return d == ST_F32 ? 4 : 2; }

/* Opens one shard and appends its tensors to the bundle's table. On error the
 * file is closed and nothing is appended. */
static cujev_status open_file(st_bundle *b, const char *path, int *cap) {
    st_file *f = (st_file *)calloc(1, sizeof *f);
    if (!f)
        return cujev_raise(CUJEV_ERR_OOM, "st_file");
    f->fd = open(path, O_RDONLY);
    cujev_status s = CUJEV_OK;
    int appended = 0;
    if (f->fd < 0) {
        s = cujev_raise(CUJEV_ERR_IO, "open %s failed", path);
        goto fail;
    }
    struct stat stt;
    if (fstat(f->fd, &stt) != 0 || stt.st_size < 8) {
        s = cujev_raise(CUJEV_ERR_FORMAT, "%s: too small", path);
        goto fail;
    }
    f->size = (size_t)stt.st_size;
    f->map = mmap(NULL, f->size, PROT_READ, MAP_PRIVATE, f->fd, 0);
    if (f->map == MAP_FAILED) {
        f->map = NULL;
        s = cujev_raise(CUJEV_ERR_IO, "mmap %s failed", path);
        goto fail;
    }
    uint64_t hlen;
    memcpy(&hlen, f->map, 8);
    if (hlen > f->size - 8) {
        s = cujev_raise(CUJEV_ERR_FORMAT, "%s: bad header length", path);
        goto fail;
    }
    {
        char err[256];
        f->header = js_parse((const char *)f->map + 8, (size_t)hlen, err, sizeof err);
        if (!f->header || !js_is(js_root(f->header), JS_OBJ)) {
            s = cujev_raise(CUJEV_ERR_FORMAT, "%s: header is not a JSON object", path);
            goto fail;
        }
    }
    {
        const char *base = (const char *)f->map + 8 + hlen;
        const size_t data_size = f->size - 8 - (size_t)hlen;
        for (const js_node *e = js_root(f->header)->child; e; e = e->next) {
            if (strcmp(e->key, "__metadata__") == 0)
                continue;
            const js_node *dt = js_get(e, "dtype"), *sh = js_get(e, "shape"),
                          *off = js_get(e, "data_offsets");
            if (!js_is(dt, JS_STR) || !js_is(sh, JS_ARR) || !js_is(off, JS_ARR) ||
                off->count != 2 || sh->count > 8) {
                s = cujev_raise(CUJEV_ERR_FORMAT, "%s: malformed entry %s", path, e->key);
                goto fail;
            }
            st_tensor t;
            memset(&t, 0, sizeof t);
            t.name = e->key;
            t.dtype = parse_dtype(dt->str);
            t.ndim = sh->count;
            size_t numel = 1;
            int i = 0;
            for (const js_node *d = sh->child; d; d = d->next, i++) {
                if (!js_is(d, JS_NUM) || d->num < 0) {
                    s = cujev_raise(CUJEV_ERR_FORMAT, "%s: bad shape of %s", path, e->key);
                    goto fail;
                }
                t.shape[i] = (int64_t)d->num;
                numel *= (size_t)t.shape[i];
            }
            t.numel = numel;
            const js_node *o0 = js_at(off, 0), *o1 = js_at(off, 1);
            if (!js_is(o0, JS_NUM) || !js_is(o1, JS_NUM) || o0->num < 0 || o1->num < o0->num ||
                (size_t)o1->num > data_size) {
                s = cujev_raise(CUJEV_ERR_FORMAT, "%s: tensor %s offsets out of range", path, e->key);
                goto fail;
            }
            t.data = base + (size_t)o0->num;
            t.nbytes = (size_t)o1->num - (size_t)o0->num;
            if (t.dtype != ST_OTHER && t.nbytes != numel * dtype_size(t.dtype)) {
                s = cujev_raise(CUJEV_ERR_FORMAT, "%s: tensor %s size does not match its shape",
                               path, e->key);
                goto fail;
            }
            if (b->num_tensors == *cap) {
                int nc = *cap ? *cap * 2 : 256;
                st_tensor *nt = (st_tensor *)realloc(b->tensors, (size_t)nc * sizeof(st_tensor));
                if (!nt) {
                    s = cujev_raise(CUJEV_ERR_OOM, "tensor table");
                    goto fail;
                }
                b->tensors = nt;
                *cap = nc;
            }
            b->tensors[b->num_tensors++] = t;
            appended++;
        }
    }
    {
        st_file **nf = (st_file **)realloc(b->files, (size_t)(b->num_files + 1) * sizeof(st_file *));
        if (!nf) {
            s = cujev_raise(CUJEV_ERR_OOM, "file table");
            goto fail;
        }
        b->files = nf;
        b->files[b->num_files++] = f;
    }
    return CUJEV_OK;
fail:
    b->num_tensors -= appended;
    st_file_close(f);
    return s;
}

cujev_status st_bundle_open(const char *dir, st_bundle *b) {
    memset(b, 0, sizeof *b);
    DIR *d = opendir(dir);
    if (!d)
        return cujev_raise(CUJEV_ERR_IO, "cannot open directory %s", dir);
    int cap = 0, nfound = 0;
    cujev_status s = CUJEV_OK;
    struct dirent *de;
    while ((de = readdir(d)) != NULL) {
        size_t L = strlen(de->d_name);
        if (L <= 12 || strcmp(de->d_name + L - 12, ".safetensors") != 0)
            continue;
        char path[4096];
        snprintf(path, sizeof path, "%s/%s", dir, de->d_name);
        nfound++;
        if ((s = open_file(b, path, &cap)) != CUJEV_OK)
            break;
    }
    closedir(d);
    if (s == CUJEV_OK && nfound == 0)
        s = cujev_raise(CUJEV_ERR_IO, "no *.safetensors in %s", dir);
    if (s != CUJEV_OK) {
        st_bundle_release(b);
        return s;
    }
    /* index: linear probing in a table at most half full */
    uint32_t nslots = 16;
    while (nslots < 2u * (uint32_t)b->num_tensors)
        nslots <<= 1;
    b->slots = (int32_t *)malloc(nslots * sizeof(int32_t));
    if (!b->slots) {
        st_bundle_release(b);
        return cujev_raise(CUJEV_ERR_OOM, "tensor index");
    }
    memset(b->slots, 0xff, nslots * sizeof(int32_t));
    b->slot_mask = nslots - 1;
    for (int i = 0; i < b->num_tensors; i++) {
        uint32_t k = name_hash(b->tensors[i].name) & b->slot_mask;
        for (; b->slots[k] >= 0; k = (k + 1) & b->slot_mask)
            if (strcmp(b->tensors[b->slots[k]].name, b->tensors[i].name) == 0) {
                s = cujev_raise(CUJEV_ERR_FORMAT, "tensor %s appears twice", b->tensors[i].name);
                st_bundle_release(b);
                return s;
            }
        b->slots[k] = i;
    }
    return CUJEV_OK;
}

void st_bundle_release(st_bundle *b) {
    for (int i = 0; i < b->num_files; i++)
        st_file_close(b->files[i]);
    free(b->files);
    free(b->tensors);
    free(b->slots);
    memset(b, 0, sizeof *b);
}

const st_tensor *st_lookup(const st_bundle *b, const char *name) {
    if (!b->slots)
        return NULL;
    for (uint32_t k = name_hash(name) & b->slot_mask; b->slots[k] >= 0; k = (k + 1) & b->slot_mask)
        if (strcmp(b->tensors[b->slots[k]].name, name) == 0)
            return &b->tensors[b->slots[k]];
    return NULL;
}
