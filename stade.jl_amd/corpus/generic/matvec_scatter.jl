# matvec_scatter(loss, a, x, y, i_m, i_n)
#
# y += A x with the matrix read as one flat loop over its column-major elements, so each
# iteration adds into a row of y that other iterations share (a scatter in the primal and a
# second one into xb in the adjoint), then loss += sum(y .^ 2).
#
# loss: length-1 output, accumulated; a: A flattened, i_m x i_n column-major; x: length i_n;
# y: length i_m, accumulated; i_m, i_n: dimensions of A
function matvec_scatter(loss, a, x, y, i_m, i_n)
    for idx = 1:i_m * i_n
        i = mod(idx - 1, i_m) + 1
        j = div(idx - 1, i_m) + 1
        y[i] = y[i] + a[idx] * x[j]
    end
    for k = 1:i_m
        loss[1] = loss[1] + y[k] ^ 2
    end
    return nothing
end
