//! hip_context.zig -- the device context of the MI355X library, in place of src/backend/cuda/cuda_context.zig.
//!
//! Same externs and the same CudaContext surface (instance / deviceCount / deviceInfo / sync / usedMemory) as
//! cuda_context.zig:1-60, bound to the hip_ functions of include/llmgen_attn.h.  The cuda_graph_* names that
//! cuda.zig:26-29 re-exports for executor.zig's captureGraphs are provided as aliases of the hip_graph_* externs,
//! so the executor needs no change.  Not compiled here (no Zig toolchain); tests/test_zig_binding.py checks the
//! externs against the C header.
pub extern fn hip_init(ws_bytes: usize) c_int;
pub extern fn hip_sync() void;
pub extern fn hip_last_error() c_int;

pub extern fn hip_graph_begin() c_int;
pub extern fn hip_graph_end() ?*anyopaque;
pub extern fn hip_graph_launch(exec: ?*anyopaque) void;
pub extern fn hip_graph_destroy(exec: ?*anyopaque) void;

pub extern fn hip_device_count() c_int;
pub extern fn hip_mem_info(free_mem: *usize, total_mem: *usize) void;
pub extern fn hip_device_info(dev: c_int, name: [*c]u8, name_cap: c_int, total_mem: *usize, arch: *c_int) void;

// memory helpers (src/backend/cuda/memory/memory.zig:1-11)
pub extern fn hip_malloc(bytes: usize) ?*anyopaque;
pub extern fn hip_free(p: ?*anyopaque) void;
pub extern fn hip_host_alloc(bytes: usize) ?*anyopaque;
pub extern fn hip_host_free(p: ?*anyopaque) void;
pub extern fn hip_h2d(dst_dev: ?*anyopaque, src_host: ?*const anyopaque, bytes: usize) void;
pub extern fn hip_d2h(dst_host: ?*anyopaque, src_dev: ?*const anyopaque, bytes: usize) void;
pub extern fn hip_d2d(dst_dev: ?*anyopaque, src_dev: ?*const anyopaque, bytes: usize) void;
pub extern fn hip_h2d_async(dst_dev: ?*anyopaque, src_host: ?*const anyopaque, bytes: usize) void;
pub extern fn hip_d2h_async(dst_host: ?*anyopaque, src_dev: ?*const anyopaque, bytes: usize) void;

// the names the executor's graph capture uses (cuda.zig:26-29)
pub const cuda_graph_begin = hip_graph_begin;
pub const cuda_graph_end = hip_graph_end;
pub const cuda_graph_launch = hip_graph_launch;
pub const cuda_graph_destroy = hip_graph_destroy;

pub const CudaContext = struct {
    inited: bool = false,

    var g_inst: ?CudaContext = null;

    /// Creates the library's stream on device 0 once.  The library has no workspace of its own (the size is
    /// accepted for the reference's signature and unused).
    pub fn instance() *CudaContext {
        if (g_inst == null) {
            _ = hip_init(0);
            g_inst = .{ .inited = true };
        }
        return &g_inst.?;
    }

    pub fn deviceCount(_: *CudaContext) i32 {
        return @intCast(hip_device_count());
    }

    /// `sm` receives the gfx number (950 for MI355X) where the CUDA build reports the SM version.
    pub fn deviceInfo(_: *CudaContext, dev: i32, name_buf: []u8) struct { total_mem: usize, sm: i32 } {
        var total: usize = 0;
        var arch: c_int = 0;
        hip_device_info(@intCast(dev), name_buf.ptr, @intCast(name_buf.len), &total, &arch);
        return .{ .total_mem = total, .sm = @intCast(arch) };
    }

    pub fn sync(_: *CudaContext) void {
        hip_sync();
    }

    /// Device memory in use (total - free on the current device), including the runtime and other processes.
    pub fn usedMemory(_: *CudaContext) usize {
        var free_mem: usize = 0;
        var total_mem: usize = 0;
        hip_mem_info(&free_mem, &total_mem);
        return total_mem - free_mem;
    }
};
