// MI355X backend of SimdYolo over libsimdyolo_hip: the HIP counterpart of
// VulkanBackend for the reference's backend contracts —
//   IComputeBackend     (Compute.cs:11-25)      host MatMul
//   IConvolutionBackend (Compute.cs:27-41)      host NCHW Conv
//   IDeviceBackend      (DeviceExecution.cs:4-76) frames, Compute, DeviceConv,
//                                               DeviceMatMul, DeviceConcat, DeviceSlice
//   IFastPathBackend    (IFastPathBackend.cs)   end-to-end top-k, joined head decode
//
// NOT BUILT IN THIS REPOSITORY: the image has no .NET SDK.  Source for the
// reference's src/SimdYolo/, compiled there with AllowUnsafeBlocks.
//
// Memory model.  Device tensors of a frame live in the library's frame arena
// (sy_frame_alloc, 256-byte aligned, reset by sy_frame_begin); constants
// (weights, IsConstant tensors) are uploaded once into persistent device
// memory (sy_malloc) and kept until Dispose.  A DeviceStorage's Buffer is the
// base device pointer (boxed nint) and Offset a byte offset into it, so
// DeviceSlice can hand out views without copies.  Tensors are dense row-major
// (NCHW for 4-d), as the reference's device tensors; the library's own
// convolution kernels run channels-last, so DeviceConv brackets sy_conv_run
// with two tensor.comp transposes (the fused whole-model path, sy_model_*,
// keeps activations channels-last end to end and needs none).
//
// Threading.  One frame at a time per backend: BeginFrame takes the monitor
// and EndFrame releases it, as VulkanExecution.cs:40-87.
//
// Replay (VulkanReplay.cs:31-129, on hipGraphs).  A frame is a replay
// candidate while its only host upload is the input BeginReplayCapture names
// and nothing non-constant is read back before its outputs.  The input is
// uploaded first in every candidate frame, so frames of one shape allocate
// from the frame arena in one order and get the same addresses.  The first
// candidate frame of a shape runs eagerly (convolutions tune, scratch grows)
// and marks the shape replayable; the next one is captured from its first op
// to its outputs (sy_graph_begin / sy_graph_end) and launched once; later
// calls of the shape (TryReplay) copy the input into the captured upload
// buffer, launch the graph and download the outputs, without a frame.  A
// captured frame that needs the host (an upload, a read-back, or a call the
// library refuses under capture with status SY_ESTATE) ends its capture
// there: the recorded work is launched once and the frame goes on op by op.
// SIMDYOLO_HIP_REPLAY=0 turns replay off, as SIMDYOLO_VULKAN_REPLAY does.
//
// Whole model.  TryRunModel hands a PtModel that HipWholeModel recognises to
// the library's native forward (sy_model_*), which is the benchmarked path;
// everything else runs through the members above.
using System.Runtime.InteropServices;

namespace SimdYolo;

// Members of the internal interfaces are implemented explicitly: their
// signatures use the reference's internal types (DeviceStorage,
// DetectionHeadLevel, CpuTensorPool).
public sealed unsafe class HipBackend : IComputeBackend, IConvolutionBackend, IDeviceBackend, IFastPathBackend
{
    private readonly object gate = new();
    private nint ctx;
    private bool disposed, frameActive;
    private long frameId;
    private readonly Dictionary<Tensor, nint> constants = new(ReferenceEqualityComparer.Instance);
    private readonly Dictionary<Tensor, DeviceStorage> frameInputs = new(ReferenceEqualityComparer.Instance);
    private readonly Dictionary<ConvKey, ulong> convolutions = [];
    private readonly Dictionary<PtModel, HipWholeModel?> wholeModels = new(ReferenceEqualityComparer.Instance);

    private const int StatusState = 5;  // SY_ESTATE: not allowed in the current state (e.g. under capture)
    private readonly bool replayEnabled = Environment.GetEnvironmentVariable("SIMDYOLO_HIP_REPLAY") != "0";
    private bool replayCandidate, capturing, uploadReading;
    private Tensor? replayInput;
    private DeviceStorage? replayUpload;
    private int[]? replayableShape;
    private ReplayPlan? replayPlan;
    private long replayedFrames;

    private sealed record ReplayOutput(nint Address, int Length, int[] Shape, int Alias);
    private sealed record ReplayPlan(int[] InputShape, int InputLength, nint InputAddress, ulong Graph, ReplayOutput[] Outputs);

    private readonly record struct ConvKey(Tensor Weights, Tensor? Bias, int Sh, int Sw, int Pt, int Pl, int Pb, int Pr,
        int Dh, int Dw, int Groups, bool Silu);

    /// <summary>Opens a context on HIP device <paramref name="device"/> (one stream, one frame arena).</summary>
    public HipBackend(int device = 0) => HipNative.Check(HipNative.Create(device, out ctx));

    public string Name => Marshal.PtrToStringUTF8(HipNative.Name(ctx)) ?? "HIP";

    long IFastPathBackend.ReplayedFrames => replayedFrames;

    public void Dispose()
    {
        lock (gate)
        {
            if (disposed) return;
            disposed = true;
            foreach (var whole in wholeModels.Values) whole?.Dispose();
            wholeModels.Clear();
            InvalidateReplay();
            foreach (nint p in constants.Values) HipNative.Free(ctx, p);
            constants.Clear();
            HipNative.Destroy(ctx);
            ctx = 0;
        }
    }

    // ================================================================ frames

    bool IDeviceBackend.FrameActive => frameActive;
    long IDeviceBackend.FrameId => frameId;

    void IDeviceBackend.BeginFrame()
    {
        Monitor.Enter(gate);
        try
        {
            ObjectDisposedException.ThrowIf(disposed, this);
            if (frameActive) throw new InvalidOperationException("An inference is already recording.");
            HipNative.Check(HipNative.FrameBegin(ctx, out frameId));
            frameActive = true;
            frameInputs.Clear();
            DeviceScope.Current = this;
        }
        catch { frameActive = false; DeviceScope.Current = null; Monitor.Exit(gate); throw; }
    }

    void IDeviceBackend.EndFrame()
    {
        try
        {
            if (!frameActive) return;
            if (capturing) AbortCapture();
            HipNative.Check(HipNative.FrameEnd(ctx));
        }
        finally
        {
            frameActive = false; DeviceScope.Current = null; frameInputs.Clear();
            replayCandidate = false; replayInput = null; replayUpload = null;
            Monitor.Exit(gate);
        }
    }

    // A status the library returns under capture for work that needs the host
    // or an allocation: end the capture (its work runs once) and report that
    // the call must be made again, eagerly.
    private bool Retry(int status)
    {
        if (status == StatusState && capturing) { AbortCapture(); return true; }
        HipNative.Check(status);
        return false;
    }

    void IDeviceBackend.ObserveHostData(Tensor tensor)
    {
        // Only shape-dependent host work keeps a frame replayable; reading a
        // non-constant value may change what the frame does next.
        if (!replayCandidate || uploadReading || tensor.IsConstant) return;
        replayCandidate = false;
        if (capturing) AbortCapture();
    }

    void IDeviceBackend.Flush()
    {
        if (capturing) AbortCapture();  // a stream wait cannot be captured
        HipNative.Check(HipNative.Flush(ctx));
    }

    float[] IDeviceBackend.Download(DeviceStorage storage)
    {
        if (!ReferenceEquals(storage.Owner, this) || !frameActive || storage.FrameId != frameId)
            throw new InvalidOperationException("Device output belongs to another inference.");
        if (capturing) AbortCapture();
        var values = GC.AllocateUninitializedArray<float>(storage.Length);
        if (values.Length > 0)
            fixed (float* host = values)
                HipNative.Check(HipNative.Memcpy(ctx, (nint)host, Address(storage), (nuint)values.Length * sizeof(float), 1));
        return values;
    }

    private static nint Address(DeviceStorage s) => (nint)s.Buffer + (nint)s.Offset;

    private Tensor AllocateTensor(int[] shape)
    {
        int length = Tensor.Count(shape);
        SyTensor view;
        if (Retry(HipNative.FrameAlloc(ctx, 1, 1, 1, Math.Max(1, length), out view)))
            HipNative.Check(HipNative.FrameAlloc(ctx, 1, 1, 1, Math.Max(1, length), out view));
        return new(new DeviceStorage(this, view.Data, 0, length, frameId), shape);
    }

    private DeviceStorage Upload(Tensor tensor)
    {
        if (tensor.Storage is { } existing && ReferenceEquals(existing.Owner, this) && existing.FrameId == frameId) return existing;
        if (frameInputs.TryGetValue(tensor, out var same)) return same;
        float[] data;
        uploadReading = true;
        try { data = tensor.Data; } finally { uploadReading = false; }
        nuint bytes = (nuint)data.Length * sizeof(float);
        DeviceStorage storage;
        if (tensor.IsConstant)
        {
            if (!constants.TryGetValue(tensor, out nint p))
            {
                if (capturing) AbortCapture();  // a device allocation and a host copy
                HipNative.Check(HipNative.Malloc(ctx, Math.Max(bytes, 4), out p));
                constants[tensor] = p;
                if (bytes > 0) fixed (float* host = data) HipNative.Check(HipNative.Memcpy(ctx, p, (nint)host, bytes, 0));
            }
            storage = new DeviceStorage(this, p, 0, data.Length, frameId);
        }
        else
        {
            // A second host upload in a frame makes it unreplayable.
            if (replayCandidate && !ReferenceEquals(tensor, replayInput)) replayCandidate = false;
            if (capturing) AbortCapture();
            HipNative.Check(HipNative.FrameAlloc(ctx, 1, 1, 1, Math.Max(1, data.Length), out var view));
            if (bytes > 0) fixed (float* host = data) HipNative.Check(HipNative.Memcpy(ctx, view.Data, (nint)host, bytes, 0));
            storage = new DeviceStorage(this, view.Data, 0, data.Length, frameId);
        }
        frameInputs[tensor] = storage;
        return storage;
    }

    // Runs host-facing work (IComputeBackend / IConvolutionBackend) inside a
    // frame: the caller's, or a private one.
    private void WithFrame(Action<HipBackend> body)
    {
        var device = (IDeviceBackend)this;
        if (frameActive && Monitor.IsEntered(gate)) { body(this); return; }
        device.BeginFrame();
        try { body(this); HipNative.Check(HipNative.Flush(ctx)); }
        finally { device.EndFrame(); }
    }

    // ================================================================ generic ops

    Tensor IDeviceBackend.Compute(int operation, Tensor[] inputs, int[] shape, uint[] parameters, int workItems)
    {
        var output = AllocateTensor(shape);
        nint* ptrs = stackalloc nint[3];
        nuint* lengths = stackalloc nuint[3];
        for (int i = 0; i < 3; i++)
        {
            ptrs[i] = 0; lengths[i] = 0;
            if (i < inputs.Length)
            {
                var s = Upload(inputs[i]);
                ptrs[i] = Address(s);
                lengths[i] = (nuint)Math.Max(1, s.Length);
            }
        }
        // Offsets are folded into the pointers: slots 28..31 stay zero.  Slot
        // 27 (bias bound) is set by the library from inputs[2].
        uint* p = stackalloc uint[32];
        for (int i = 0; i < 32; i++) p[i] = i < parameters.Length && i < 27 ? parameters[i] : 0u;
        if (Retry(HipNative.Compute(ctx, operation, ptrs, lengths, p, workItems, Address(output.Storage!),
                (nuint)Math.Max(1, output.Length))))
            HipNative.Check(HipNative.Compute(ctx, operation, ptrs, lengths, p, workItems, Address(output.Storage!),
                (nuint)Math.Max(1, output.Length)));
        return output;
    }

    Tensor IDeviceBackend.DeviceMatMul(Tensor a, Tensor b, int[] shape)
    {
        if (a.Rank < 2 || b.Rank < 2) throw new ArgumentException("Device MatMul needs matrices.");
        int m = a.Shape[^2], k = a.Shape[^1], n = b.Shape[^1];
        if (b.Shape[^2] != k) throw new ArgumentException("MatMul inner dimensions differ.");
        if (m == 0 || n == 0 || k == 0) throw new NotSupportedException("Empty device MatMul.");
        int rank = shape.Length - 2;
        if (rank > 4) throw new NotSupportedException("Device MatMul batch rank > 4.");
        int* batch = stackalloc int[4];
        long* aStrides = stackalloc long[4];
        long* bStrides = stackalloc long[4];
        BatchStrides(a.Shape, shape, rank, aStrides);
        BatchStrides(b.Shape, shape, rank, bStrides);
        for (int j = 0; j < rank; j++) batch[j] = shape[j];
        var sa = Upload(a); var sb = Upload(b); var output = AllocateTensor(shape);
        // The MFMA route transposes B into the context scratch, which may have to grow: under capture that
        // is refused (SY_ESTATE), the capture ends and the product runs eagerly.
        if (Retry(HipNative.MatMul(ctx, Address(sa), Address(sb), Address(output.Storage!), m, n, k, rank, batch,
                aStrides, bStrides, (nuint)sa.Length, (nuint)sb.Length, (nuint)output.Length)))
            HipNative.Check(HipNative.MatMul(ctx, Address(sa), Address(sb), Address(output.Storage!), m, n, k, rank, batch,
                aStrides, bStrides, (nuint)sa.Length, (nuint)sb.Length, (nuint)output.Length));
        return output;
    }

    // Matrix strides of an operand per output batch axis (numpy broadcasting:
    // operand batch axes align to the right; size-1 axes broadcast with 0).
    private static void BatchStrides(int[] operand, int[] output, int rank, long* strides)
    {
        int own = operand.Length - 2;
        long acc = 1;
        for (int j = rank - 1; j >= 0; j--)
        {
            int d = j - (rank - own);
            int size = d >= 0 ? operand[d] : 1;
            strides[j] = size == 1 ? 0 : acc;
            if (size != 1 && size != output[j]) throw new ArgumentException("MatMul batch dimensions do not broadcast.");
            acc *= size;
        }
    }

    Tensor IDeviceBackend.DeviceConcat(IReadOnlyList<Tensor> tensors, int axis, int[] shape)
    {
        var output = AllocateTensor(shape);
        if (output.Length == 0) return output;
        int inner = Tensor.Count(shape[(axis + 1)..]);
        uint start = 0;
        uint* p = stackalloc uint[32];
        nint* ptrs = stackalloc nint[3];
        nuint* lengths = stackalloc nuint[3];
        foreach (var tensor in tensors)
        {
            if (tensor.Length == 0) continue;
            var source = Upload(tensor);
            // tensor.comp op 26 writes this input at its axis offset (VulkanExecution.cs:440-452).
            for (int i = 0; i < 32; i++) p[i] = 0;
            p[0] = (uint)tensor.Length; p[1] = (uint)tensor.Shape[axis]; p[2] = (uint)shape[axis]; p[3] = (uint)inner; p[4] = start;
            ptrs[0] = Address(source); lengths[0] = (nuint)source.Length;
            ptrs[1] = ptrs[2] = 0; lengths[1] = lengths[2] = 0;
            if (Retry(HipNative.Compute(ctx, 26, ptrs, lengths, p, tensor.Length, Address(output.Storage!), (nuint)output.Length)))
                HipNative.Check(HipNative.Compute(ctx, 26, ptrs, lengths, p, tensor.Length, Address(output.Storage!), (nuint)output.Length));
            start += (uint)tensor.Shape[axis];
        }
        return output;
    }

    Tensor IDeviceBackend.DeviceSlice(Tensor x, int[] shape, int axis, int start)
    {
        var source = Upload(x);
        int inner = Tensor.Count(x.Shape[(axis + 1)..]), outer = Tensor.Count(x.Shape[..axis]);
        // A leading-axis slice is contiguous: borrow it (any 4-byte offset is a valid HIP pointer).
        if (outer == 1)
            return new(new DeviceStorage(this, source.Buffer, source.Offset + (ulong)start * (ulong)inner * sizeof(float),
                Tensor.Count(shape), frameId), shape);
        return ((IDeviceBackend)this).Compute(24, [x], shape, DeviceOps.Parameters((uint)Tensor.Count(shape),
            (uint)x.Shape[axis], (uint)shape[axis], (uint)inner, (uint)start), Tensor.Count(shape));
    }

    // ================================================================ convolution

    private ulong Convolution(Tensor w, Tensor? bias, int[] stride, int[] pads, int[] dilation, int groups, bool silu)
    {
        if (!w.IsConstant || (bias is not null && !bias.IsConstant))
            throw new NotSupportedException("HIP convolutions pack constant weights once; computed weights are not supported.");
        var key = new ConvKey(w, bias, stride[0], stride[1], pads[0], pads[1], pads[2], pads[3], dilation[0], dilation[1], groups, silu);
        if (convolutions.TryGetValue(key, out ulong conv)) return conv;
        if (capturing) AbortCapture();  // packing weights allocates
        int oc = w.Shape[0], ic = w.Shape[1] * groups, kh = w.Shape[2], kw = w.Shape[3];
        fixed (float* wp = w.Data)
        fixed (float* bp = bias?.Data)
            HipNative.Check(HipNative.ConvCreate(ctx, wp, bp, oc, ic, kh, kw, stride[0], stride[1], pads[0], pads[1], pads[2],
                pads[3], dilation[0], dilation[1], groups, silu ? 1 : 0, out conv));
        convolutions[key] = conv;
        return conv;
    }

    private static SyTensor View(nint data, int n, int c, int h, int w) =>
        new() { Data = data, N = n, C = c, H = h, W = w, Ldc = c, Layout = HipNative.LayoutNhwc };

    Tensor IDeviceBackend.DeviceConv(Tensor x, Tensor w, Tensor? bias, int[] shape, int[] stride, int[] pads, int[] dilation,
        int groups, bool silu)
    {
        ulong conv = Convolution(w, bias, stride, pads, dilation, groups, silu);
        int n = x.Shape[0], ic = x.Shape[1], h = x.Shape[2], wd = x.Shape[3], oc = shape[1], oh = shape[2], ow = shape[3];
        var nhwc = DeviceOps.Transpose(this, x, [0, 2, 3, 1], [n, h, wd, ic]);
        var y = AllocateTensor([n, oh, ow, oc]);
        // A conv shape seen for the first time tunes (times candidates with events) and may grow the
        // scratch: under capture the library refuses that, and the conv runs after the capture ends.
        if (Retry(HipNative.ConvRun(ctx, conv, View(Address(nhwc.Storage!), n, ic, h, wd),
                View(Address(y.Storage!), n, oc, oh, ow), null)))
            HipNative.Check(HipNative.ConvRun(ctx, conv, View(Address(nhwc.Storage!), n, ic, h, wd),
                View(Address(y.Storage!), n, oc, oh, ow), null));
        return DeviceOps.Transpose(this, y, [0, 3, 1, 2], shape);
    }

    public void Conv(Tensor input, Tensor weights, Tensor? bias, Tensor output, int[] strides, int[] pads, int[] dilation,
        int groups, bool silu)
    {
        if (input.Rank != 4 || output.Rank != 4) throw new ArgumentException("Conv requires NCHW tensors.");
        WithFrame(self =>
        {
            ulong conv = self.Convolution(weights, bias, strides, pads, dilation, groups, silu);
            int n = input.Shape[0], ic = input.Shape[1], h = input.Shape[2], w = input.Shape[3];
            int oc = output.Shape[1], oh = output.Shape[2], ow = output.Shape[3];
            HipNative.Check(HipNative.FrameAlloc(self.ctx, n, ic, h, w, out var x));
            HipNative.Check(HipNative.FrameAlloc(self.ctx, n, oc, oh, ow, out var y));
            fixed (float* src = input.Data) HipNative.Check(HipNative.UploadNchw(self.ctx, src, x));
            HipNative.Check(HipNative.ConvRun(self.ctx, conv, x, y, null));
            fixed (float* dst = output.Data) HipNative.Check(HipNative.DownloadNchw(self.ctx, y, dst));
        });
    }

    public void MatMul(float[] a, float[] b, float[] c, int m, int n, int k)
    {
        if (a.Length < (long)m * k || b.Length < (long)k * n || c.Length < (long)m * n) throw new ArgumentException("MatMul buffers are too small.");
        WithFrame(self =>
        {
            HipNative.Check(HipNative.FrameAlloc(self.ctx, 1, 1, 1, Math.Max(1, m * k), out var da));
            HipNative.Check(HipNative.FrameAlloc(self.ctx, 1, 1, 1, Math.Max(1, k * n), out var db));
            HipNative.Check(HipNative.FrameAlloc(self.ctx, 1, 1, 1, Math.Max(1, m * n), out var dc));
            fixed (float* pa = a) HipNative.Check(HipNative.Memcpy(self.ctx, da.Data, (nint)pa, (nuint)(m * k) * sizeof(float), 0));
            fixed (float* pb = b) HipNative.Check(HipNative.Memcpy(self.ctx, db.Data, (nint)pb, (nuint)(k * n) * sizeof(float), 0));
            HipNative.Check(HipNative.MatMul(self.ctx, da.Data, db.Data, dc.Data, m, n, k, 0, null, null, null,
                (nuint)(m * k), (nuint)(k * n), (nuint)(m * n)));
            fixed (float* pc = c) HipNative.Check(HipNative.Memcpy(self.ctx, (nint)pc, dc.Data, (nuint)(m * n) * sizeof(float), 1));
        });
    }

    // ================================================================ fast paths

    Tensor? IFastPathBackend.TryEndToEndTopK(Tensor input, int maximum, int classes) => TopK(input, null, maximum, classes, false);

    Tensor? IFastPathBackend.TryEndToEndTopKWithExtras(Tensor input, Tensor extras, int maximum, int classes) =>
        TopK(input, extras, maximum, classes, false);

    Tensor? IFastPathBackend.TryEndToEndTopKOnnx(Tensor input, int maximum, int classes) => TopK(input, null, maximum, classes, true);

    // Two-stage top-k on the device (sy_e2e_topk), output [batch, k, 6 + extra]
    // as VulkanTopK.cs:30-70.  Extras given as a separate [batch, extra,
    // anchors] tensor are joined behind the head rows first (op 26), since the
    // library reads them inline.  Requests beyond the library's limits return
    // null, and the caller takes the reference's CPU selection.
    private Tensor? TopK(Tensor input, Tensor? extras, int maximum, int classes, bool onnx)
    {
        if (!frameActive || input.Rank != 3 || input.Shape[1] < classes + 4 || classes <= 0 || maximum <= 0) return null;
        int batch = input.Shape[0], anchors = input.Shape[2], k = Math.Min(maximum, anchors);
        if (k > 1024 || (long)k * classes > 32768 || anchors > 16_777_216) return null;
        Tensor head = input;
        if (extras is not null)
        {
            if (input.Shape[1] != classes + 4 || extras.Rank != 3 || extras.Shape[0] != batch || extras.Shape[2] != anchors) return null;
            head = ((IDeviceBackend)this).DeviceConcat([input, extras], 1, [batch, classes + 4 + extras.Shape[1], anchors]);
        }
        var source = Upload(head);
        int fields = 6 + head.Shape[1] - classes - 4;
        var output = AllocateTensor([batch, k, fields]);
        // Under capture the allocation-free form runs (the context scratch cannot grow there).
        if (capturing)
            HipNative.Check(HipNative.EndToEndTopKNoAlloc(ctx, Address(source), batch, head.Shape[1], anchors, classes, maximum,
                onnx ? 1 : 0, Address(output.Storage!)));
        else
            HipNative.Check(HipNative.EndToEndTopK(ctx, Address(source), batch, head.Shape[1], anchors, classes, maximum,
                onnx ? 1 : 0, Address(output.Storage!)));
        return output;
    }

    // Per-level op 30 into the joined [batch, nc + 4, total] output, each level
    // at its anchor offset (the multi-level decode of VulkanExecution.cs:295-324).
    Tensor IFastPathBackend.DecodeHeadLevels(DetectionHeadLevel[] levels, int[] shape, int bins, bool xyxy)
    {
        var output = AllocateTensor(shape);
        int total = shape[2], start = 0;
        uint* p = stackalloc uint[32];
        nint* ptrs = stackalloc nint[3];
        nuint* lengths = stackalloc nuint[3];
        foreach (var level in levels)
        {
            int n = level.Boxes.Shape[0], h = level.Boxes.Shape[2], w = level.Boxes.Shape[3], nc = level.Scores.Shape[1];
            var boxes = Upload(level.Boxes); var scores = Upload(level.Scores);
            for (int i = 0; i < 32; i++) p[i] = 0;
            p[0] = (uint)(n * h * w); p[1] = (uint)(h * w); p[2] = (uint)w; p[3] = (uint)bins; p[4] = (uint)nc;
            p[5] = DeviceOps.Bits(level.Stride); p[6] = xyxy ? 1u : 0u; p[7] = (uint)total; p[8] = (uint)start;
            ptrs[0] = Address(boxes); lengths[0] = (nuint)boxes.Length;
            ptrs[1] = Address(scores); lengths[1] = (nuint)scores.Length;
            ptrs[2] = 0; lengths[2] = 0;
            if (Retry(HipNative.Compute(ctx, 30, ptrs, lengths, p, n * h * w, Address(output.Storage!), (nuint)output.Length)))
                HipNative.Check(HipNative.Compute(ctx, 30, ptrs, lengths, p, n * h * w, Address(output.Storage!), (nuint)output.Length));
            start += h * w;
        }
        return output;
    }

    // ================================================================ replay

    void IFastPathBackend.BeginReplayCapture(Tensor input)
    {
        replayCandidate = replayEnabled && frameActive && input.Storage is null && input.Length > 0 && !input.IsConstant;
        replayInput = replayCandidate ? input : null;
        replayUpload = null;
        if (!replayCandidate) return;
        replayUpload = Upload(input);  // the first allocation of every candidate frame
        if (replayPlan is null && replayableShape is not null && input.Shape.AsSpan().SequenceEqual(replayableShape))
        {
            HipNative.Check(HipNative.GraphBegin(ctx));
            capturing = true;
        }
    }

    // Ends a capture before its frame does: the work recorded so far runs
    // once, and the frame continues op by op.  The shape is recorded again
    // only after another qualifying eager frame.
    private void AbortCapture()
    {
        capturing = false;
        replayCandidate = false;
        replayableShape = null;
        HipNative.Check(HipNative.GraphEnd(ctx, out ulong partial));
        HipNative.Check(HipNative.GraphLaunch(ctx, partial));
        HipNative.Check(HipNative.GraphDestroy(ctx, partial));
    }

    private void InvalidateReplay()
    {
        if (replayPlan is { } plan && ctx != 0) HipNative.GraphDestroy(ctx, plan.Graph);
        replayPlan = null;
        replayableShape = null;
    }

    // At the end of a candidate frame (its outputs are known): a captured
    // frame becomes the shape's replay plan and runs once now; an eager
    // candidate frame makes its shape replayable.
    private void CompleteFrame(Tensor[] outputs)
    {
        bool deviceOutputs = outputs.Length > 0 && outputs.All(t => t.Storage is { Length: > 0 } s && ReferenceEquals(s.Owner, this));
        if (capturing)
        {
            if (!replayCandidate || !deviceOutputs) { AbortCapture(); return; }
            capturing = false;
            HipNative.Check(HipNative.GraphEnd(ctx, out ulong graph));
            HipNative.Check(HipNative.GraphLaunch(ctx, graph));
            var descriptions = new ReplayOutput[outputs.Length];
            var aliases = new Dictionary<Tensor, int>(ReferenceEqualityComparer.Instance);
            for (int i = 0; i < outputs.Length; i++)
            {
                if (!aliases.TryGetValue(outputs[i], out int alias)) { alias = i; aliases.Add(outputs[i], i); }
                descriptions[i] = new(Address(outputs[i].Storage!), outputs[i].Length, (int[])outputs[i].Shape.Clone(), alias);
            }
            replayPlan = new((int[])replayInput!.Shape.Clone(), replayInput.Length, Address(replayUpload!), graph, descriptions);
        }
        else if (replayCandidate && deviceOutputs && replayPlan is null)
        {
            replayableShape = (int[])replayInput!.Shape.Clone();
        }
        replayCandidate = false;
    }

    // Without a frame: the input into the captured upload buffer, one graph
    // launch, the outputs into fresh host arrays (VulkanReplay.TryReplay).
    bool IFastPathBackend.TryReplay(Tensor input, out Tensor[] outputs, CpuTensorPool? outputPool)
    {
        lock (gate)
        {
            ObjectDisposedException.ThrowIf(disposed, this);
            outputs = [];
            if (replayPlan is not { } plan || frameActive || input.Storage is not null || input.IsConstant ||
                input.Length != plan.InputLength || !input.Shape.AsSpan().SequenceEqual(plan.InputShape)) return false;
            try
            {
                fixed (float* source = input.Data)
                    HipNative.Check(HipNative.Memcpy(ctx, plan.InputAddress, (nint)source, (nuint)input.Length * sizeof(float), 0));
                int status = HipNative.GraphLaunch(ctx, plan.Graph);
                if (status == StatusState) { InvalidateReplay(); return false; }  // the scratch moved since the capture
                HipNative.Check(status);
                outputs = new Tensor[plan.Outputs.Length];
                for (int i = 0; i < outputs.Length; i++)
                {
                    var d = plan.Outputs[i];
                    if (d.Alias != i) { outputs[i] = outputs[d.Alias]; continue; }
                    float[] values = outputPool?.Rent(d.Length, clear: false) ?? GC.AllocateUninitializedArray<float>(d.Length);
                    fixed (float* target = values)
                        HipNative.Check(HipNative.Memcpy(ctx, (nint)target, d.Address, (nuint)d.Length * sizeof(float), 1));
                    outputs[i] = new(values, d.Shape);
                }
                replayedFrames++;
                return true;
            }
            catch { InvalidateReplay(); throw; }
        }
    }

    void IDeviceBackend.MaterializeOutputs(Tensor[] outputs)
    {
        CompleteFrame(outputs);
        foreach (var output in outputs) _ = output.Data;
    }

    // ================================================================ whole model

    bool IFastPathBackend.TryRunModel(object model, Tensor input, CpuTensorPool? outputPool, out Tensor[] outputs)
    {
        outputs = [];
        if (model is not PtModel pt || input.Storage is not null || input.Rank != 4) return false;
        lock (gate)
        {
            ObjectDisposedException.ThrowIf(disposed, this);
            if (frameActive) return false;
            if (!wholeModels.TryGetValue(pt, out var whole))
            {
                whole = HipWholeModel.TryCreate(ctx, pt);
                wholeModels[pt] = whole;
            }
            if (whole is null) return false;
            outputs = whole.Predict(input, outputPool);
            return true;
        }
    }

    // One synchronous copy per output; the library's stream already orders them.
    void IFastPathBackend.DownloadFrameOutputs(Tensor[] outputs, CpuTensorPool? outputPool)
    {
        CompleteFrame(outputs);
        HipNative.Check(HipNative.Flush(ctx));
        foreach (var tensor in outputs)
        {
            if (tensor.Storage is not { } storage) continue;
            if (!frameActive || !ReferenceEquals(storage.Owner, this) || storage.FrameId != frameId)
                throw new InvalidOperationException("Device output belongs to another inference.");
            float[] values = outputPool?.Rent(storage.Length, clear: false) ?? GC.AllocateUninitializedArray<float>(storage.Length);
            if (storage.Length > 0)
                fixed (float* host = values)
                    HipNative.Check(HipNative.Memcpy(ctx, (nint)host, Address(storage), (nuint)storage.Length * sizeof(float), 1));
            tensor.AcceptDownloadedData(values);
        }
    }
}
