// The BASIS memory API (reference include/basis/core/memory.h:7-29, declared
// there and implemented nowhere) on HBM: an arena of hipMalloc'd blocks and
// a pool of fixed-size device objects with a host-side free list.
#include <stdlib.h>
#include <string.h>

#include <new>
#include <vector>

#include "common.hpp"
#include "lancius_basis.h"

struct basis_arena {
    struct Block {
        char* base;
        size_t size;
        size_t used;
        unsigned epoch;  // `used` counts only when it equals the arena's epoch
    };
    int device;
    size_t block_size;
    std::vector<Block> blocks;
    size_t cur;      // block being bumped
    unsigned epoch;  // incremented by reset: every block is empty again
};

struct basis_pool {
    int device;
    size_t stride;      // object size rounded up to 256 bytes
    size_t per_chunk;
    std::vector<char*> chunks;
    std::vector<char*> free_list;            // host-side stack of free objects
    std::vector<std::vector<uint8_t>> live;  // per chunk: 1 while an object is handed out
};

namespace {

constexpr size_t kAlign = 256;

size_t round_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

bool set_device(int device) {
    const hipError_t e = hipSetDevice(device);
    if (e != hipSuccess) {
        lancius::set_error(LANCIUS_HIP_ERR_INTERNAL, "basis: hipSetDevice(%d): %s", device, hipGetErrorString(e));
        return false;
    }
    return true;
}

char* device_alloc(size_t bytes, const char* what) {
    void* p = nullptr;
    const hipError_t e = hipMalloc(&p, bytes);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        lancius::set_error(e == hipErrorOutOfMemory ? LANCIUS_HIP_ERR_OOM : LANCIUS_HIP_ERR_INTERNAL,
                           "%s: hipMalloc(%zu): %s", what, bytes, hipGetErrorString(e));
        return nullptr;
    }
    return (char*)p;
}

// Offset of the first `alignment`-aligned address at or after base + used.
size_t aligned_offset(const char* base, size_t used, size_t alignment) {
    const uintptr_t a = (uintptr_t)(base + used);
    return used + (size_t)(((a + alignment - 1) & ~(uintptr_t)(alignment - 1)) - a);
}

}  // namespace

extern "C" {

basis_arena* basis_arena_create(size_t default_block_size) {
    int device = 0;
    if (hipGetDevice(&device) != hipSuccess) {
        lancius::set_error(LANCIUS_HIP_ERR_INTERNAL, "basis_arena_create: no HIP device");
        return nullptr;
    }
    basis_arena* a = new (std::nothrow) basis_arena();
    if (!a) {
        lancius::set_error(LANCIUS_HIP_ERR_OOM, "basis_arena_create: host allocation");
        return nullptr;
    }
    a->device = device;
    a->block_size = default_block_size ? round_up(default_block_size, kAlign) : ((size_t)1 << 20);
    a->cur = 0;
    a->epoch = 1;
    char* base = device_alloc(a->block_size, "basis_arena_create");
    if (!base) {
        delete a;
        return nullptr;
    }
    a->blocks.push_back({base, a->block_size, 0, a->epoch});
    return a;
}

void* basis_arena_alloc(basis_arena* a, size_t size, size_t alignment) {
    if (!a) {
        lancius::set_error(LANCIUS_HIP_ERR_NULL_PTR, "basis_arena_alloc: NULL arena");
        return nullptr;
    }
    if (alignment == 0) alignment = kAlign;
    if ((alignment & (alignment - 1)) != 0 || size > ((size_t)1 << 46)) {
        lancius::set_error(LANCIUS_HIP_ERR_SHAPE, "basis_arena_alloc: size %zu, alignment %zu", size, alignment);
        return nullptr;
    }
    // Current block, then the blocks after it (kept from before a reset),
    // then a new block.
    for (size_t i = a->cur; i < a->blocks.size(); ++i) {
        basis_arena::Block& b = a->blocks[i];
        if (b.epoch != a->epoch) {
            b.epoch = a->epoch;
            b.used = 0;
        }
        const size_t off = aligned_offset(b.base, b.used, alignment);
        if (off <= b.size && size <= b.size - off) {
            b.used = off + size;
            a->cur = i;
            return b.base + off;
        }
    }
    if (!set_device(a->device)) return nullptr;
    const size_t bytes = round_up(size + alignment > a->block_size ? size + alignment : a->block_size, kAlign);
    char* base = device_alloc(bytes, "basis_arena_alloc");
    if (!base) return nullptr;
    a->blocks.push_back({base, bytes, 0, a->epoch});
    basis_arena::Block& b = a->blocks.back();
    const size_t off = aligned_offset(b.base, 0, alignment);
    b.used = off + size;
    a->cur = a->blocks.size() - 1;
    return b.base + off;
}

void basis_arena_reset(basis_arena* a) {
    if (!a) return;
    ++a->epoch;
    a->cur = 0;
}

void basis_arena_destroy(basis_arena* a) {
    if (!a) return;
    if (set_device(a->device))
        for (basis_arena::Block& b : a->blocks) (void)hipFree(b.base);
    delete a;
}

size_t lancius_basis_arena_capacity(const basis_arena* a) {
    size_t n = 0;
    if (a)
        for (const basis_arena::Block& b : a->blocks) n += b.size;
    return n;
}

basis_pool* basis_pool_create(size_t object_size, size_t objects_per_chunk) {
    if (object_size == 0 || objects_per_chunk == 0 || object_size > ((size_t)1 << 40) ||
        objects_per_chunk > ((size_t)1 << 24)) {
        lancius::set_error(LANCIUS_HIP_ERR_SHAPE, "basis_pool_create: object_size %zu, objects_per_chunk %zu",
                           object_size, objects_per_chunk);
        return nullptr;
    }
    int device = 0;
    if (hipGetDevice(&device) != hipSuccess) {
        lancius::set_error(LANCIUS_HIP_ERR_INTERNAL, "basis_pool_create: no HIP device");
        return nullptr;
    }
    basis_pool* p = new (std::nothrow) basis_pool();
    if (!p) {
        lancius::set_error(LANCIUS_HIP_ERR_OOM, "basis_pool_create: host allocation");
        return nullptr;
    }
    p->device = device;
    p->stride = round_up(object_size, kAlign);
    p->per_chunk = objects_per_chunk;
    return p;
}

void* basis_pool_alloc(basis_pool* p) {
    if (!p) {
        lancius::set_error(LANCIUS_HIP_ERR_NULL_PTR, "basis_pool_alloc: NULL pool");
        return nullptr;
    }
    if (p->free_list.empty()) {
        if (!set_device(p->device)) return nullptr;
        char* chunk = device_alloc(p->stride * p->per_chunk, "basis_pool_alloc");
        if (!chunk) return nullptr;
        p->chunks.push_back(chunk);
        p->live.emplace_back(p->per_chunk, (uint8_t)0);
        // pushed in reverse so objects come out in address order
        for (size_t i = p->per_chunk; i-- > 0;) p->free_list.push_back(chunk + i * p->stride);
    }
    char* obj = p->free_list.back();
    p->free_list.pop_back();
    for (size_t c = 0; c < p->chunks.size(); ++c) {
        const char* base = p->chunks[c];
        if (obj >= base && obj < base + p->stride * p->per_chunk) {
            p->live[c][(size_t)(obj - base) / p->stride] = 1;
            break;
        }
    }
    return obj;
}

void basis_pool_free(basis_pool* p, void* ptr) {
    if (!p || !ptr) return;
    const char* q = (const char*)ptr;
    for (size_t c = 0; c < p->chunks.size(); ++c) {
        const char* base = p->chunks[c];
        if (q < base || q >= base + p->stride * p->per_chunk) continue;
        const size_t off = (size_t)(q - base);
        if (off % p->stride != 0) return;  // not an object start
        uint8_t& live = p->live[c][off / p->stride];
        if (!live) return;  // already free
        live = 0;
        p->free_list.push_back((char*)ptr);
        return;
    }
}

void basis_pool_destroy(basis_pool* p) {
    if (!p) return;
    if (set_device(p->device))
        for (char* c : p->chunks) (void)hipFree(c);
    delete p;
}

size_t lancius_basis_pool_capacity(const basis_pool* p) { return p ? p->chunks.size() * p->stride * p->per_chunk : 0; }

}  // extern "C"
