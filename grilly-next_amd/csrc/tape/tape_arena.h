// tape_arena.h — bump allocator holding the Wengert list of one forward pass.
//
// Same contract as the reference TapeArena (cpp/include/grilly/autograd/tape_arena.h:64-170):
// objects are placement-constructed, never destroyed individually, and reset() drops the
// whole tape in O(1).  Nodes therefore own no heap memory.  Allocation beyond the capacity
// throws std::bad_alloc (tape_arena.h:94-108).
#pragma once

#include <cstddef>
#include <cstdint>
#include <cstdlib>
#include <new>
#include <utility>

namespace grilly {
namespace autograd {

class TapeArena {
public:
    static constexpr size_t kDefaultCapacity = 64ull << 20;  // 64 MiB (tape_arena.h:69)

    explicit TapeArena(size_t capacity = kDefaultCapacity) : capacity_(capacity) {
        base_ = static_cast<uint8_t*>(std::aligned_alloc(64, round_up(capacity_ ? capacity_ : 64, 64)));
        if (!base_) throw std::bad_alloc();
    }
    ~TapeArena() { std::free(base_); }
    TapeArena(const TapeArena&) = delete;
    TapeArena& operator=(const TapeArena&) = delete;

    template <typename T, typename... Args>
    T* allocate(Args&&... args) {
        void* p = allocate_bytes(sizeof(T), alignof(T));
        return new (p) T(std::forward<Args>(args)...);
    }

    // Allocates a node and threads it onto the Wengert list (defined in autograd.h,
    // where Node is complete).
    template <typename T, typename... Args>
    T* allocate_node(Args&&... args);

    void* allocate_bytes(size_t bytes, size_t align) {
        size_t off = round_up(offset_, align);
        if (off + bytes > capacity_) throw std::bad_alloc();
        offset_ = off + bytes;
        return base_ + off;
    }

    void reset() {
        offset_ = 0;
        tail_ = nullptr;
    }

    struct Mark {
        size_t offset;
        void* tail;
    };
    Mark save() const { return {offset_, tail_}; }
    void restore(const Mark& m) {
        offset_ = m.offset;
        tail_ = m.tail;
    }

    template <typename T = void>
    T* tail() const { return static_cast<T*>(tail_); }
    void set_tail(void* t) { tail_ = t; }

    size_t bytes_used() const { return offset_; }
    size_t capacity() const { return capacity_; }
    float utilization() const { return capacity_ ? float(offset_) / float(capacity_) : 0.f; }

private:
    static size_t round_up(size_t x, size_t a) { return (x + a - 1) / a * a; }
    uint8_t* base_ = nullptr;
    size_t capacity_ = 0;
    size_t offset_ = 0;
    void* tail_ = nullptr;
};

}  // namespace autograd
}  // namespace grilly
